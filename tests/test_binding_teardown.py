"""Destroy order of the ctypes binding's objects, on the CPU: an executor's
destroy returns its slots to the pool and its pages to the KV cache
(gdn_exec_destroy), so closing the pool or the cache first must destroy the
executors registered with it first, and a closed executor must leave those
lists (so it no longer keeps the pool alive). Fake library objects record the
calls; nothing touches a GPU."""
import gdn_amd


class _Lib:
    def __init__(self, log):
        self.log = log

    def gdn_exec_destroy(self, h):
        self.log.append(("exec", h))
        return 0

    def gdn_pool_destroy(self, h):
        self.log.append(("pool", h))
        return 0

    def gdn_kv_destroy(self, h):
        self.log.append(("kv", h))
        return 0


class _Obj:
    pass


def _executor(lib, handle, owners):
    ex = _Obj()
    ex.lib, ex.handle, ex._owners = lib, handle, []
    ex._destroy = gdn_amd.Executor._destroy.__get__(ex)
    for o in owners:
        if getattr(o, "_deps", None) is None:
            o._deps = gdn_amd._Dependents()
        o._deps.add(ex)
        ex._owners.append(o._deps)
    return ex


def _owner(lib, handle, cls):
    o = _Obj()
    o.lib, o.handle = lib, handle
    o.close = cls.close.__get__(o)
    return o


def test_pool_close_destroys_its_executors_first():
    log = []
    lib = _Lib(log)
    pool, kv = _owner(lib, 7, gdn_amd.Pool), _owner(lib, 9, gdn_amd.KVCache)
    e1 = _executor(lib, 1, [pool, kv])
    e2 = _executor(lib, 2, [pool])
    pool.close()
    assert log == [("exec", 2), ("exec", 1), ("pool", 7)]
    assert e1.handle is None and e2.handle is None
    assert kv._deps.items == []      # e1 left the cache's list when it was destroyed
    kv.close()
    assert log[-1] == ("kv", 9) and len(log) == 4


def test_closed_executor_leaves_the_lists():
    log = []
    lib = _Lib(log)
    pool = _owner(lib, 7, gdn_amd.Pool)
    e = _executor(lib, 1, [pool])
    e._destroy()
    e._destroy()                     # a second close is a no-op
    assert pool._deps.items == []
    pool.close()
    assert log == [("exec", 1), ("pool", 7)]
