"""The Python binding's exit registry (ai_amd/_native.py), on the CPU: objects
that own library handles are closed at interpreter exit in reverse creation
order (a model before the context it was created on), collected ones are
forgotten, and a close() that raises does not stop the others. The GPU
side (a program that leaves its context and model open exits cleanly) is
tests/test_gpu_exit.py."""
import gc

from ai_amd import _native as N


class Owner:
    def __init__(self, name, log, fail=False):
        self.name, self.log, self.fail = name, log, fail
        N.own(self)

    def close(self):
        self.log.append(self.name)
        if self.fail:
            raise RuntimeError("close failed")


def test_closed_in_reverse_creation_order():
    saved = list(N._owners)
    N._owners.clear()
    try:
        log = []
        ctx = Owner("ctx", log)
        model = Owner("model", log, fail=True)  # a failing close must not stop the context's
        dropped = Owner("dropped", log)
        del dropped
        gc.collect()
        N._close_owners()
        assert log == ["model", "ctx"]
        assert N._owners == []
        del ctx, model
    finally:
        N._owners[:] = saved


def test_collected_owners_are_forgotten():
    saved = list(N._owners)
    N._owners.clear()
    try:
        log = []
        for i in range(100):
            Owner(f"o{i}", log)  # each dropped at once
        gc.collect()
        Owner("last", log)  # registering prunes the dead references
        assert len(N._owners) == 1
    finally:
        N._owners[:] = saved
