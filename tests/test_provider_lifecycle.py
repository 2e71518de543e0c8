"""Host-side lifetime rules of the Python provider (no device): a relation or
join index must never reach the library after its provider's context is
destroyed.  When the provider and its relations are collected in one garbage
batch (a reference cycle, or interpreter shutdown), weak references are
cleared before any finalizer runs, so close() cannot see them; their own
finalizers run afterwards and must not free through the dead context."""
import ctypes as C
import gc

import xlog_amd.provider as pv


class _FakeLib:
    def __init__(self):
        self.calls = []

    def xlog_hip_ctx_create(self, device, ref):
        ref._obj.value = 0x1000
        self.calls.append("create")
        return 0

    def xlog_hip_ctx_destroy(self, ctx):
        self.calls.append("destroy")

    def _free(self, what):
        self.calls.append((what, "after-destroy" if "destroy" in self.calls else "before-destroy"))

    def xlog_hip_rel_free(self, h):
        self._free("rel_free")

    def xlog_hip_join_index_free(self, h):
        self._free("join_index_free")


def test_handles_collected_with_their_provider(monkeypatch):
    fake = _FakeLib()
    monkeypatch.setattr(pv, "_lib", fake)
    p = pv.HipKernelProvider(0)
    rels = [p._rel(C.c_void_p(0x2000 + i)) for i in range(3)]
    ix = pv.JoinIndex(p, C.c_void_p(0x3000), [0])
    p._live.add(ix)
    p.cycle = (rels, ix)  # provider -> handles -> provider: one garbage batch
    del rels, ix, p
    gc.collect()
    assert "destroy" in fake.calls
    assert not any(isinstance(c, tuple) and c[1] == "after-destroy" for c in fake.calls), fake.calls


def test_close_frees_live_handles_first(monkeypatch):
    fake = _FakeLib()
    monkeypatch.setattr(pv, "_lib", fake)
    p = pv.HipKernelProvider(0)
    keep = [p._rel(C.c_void_p(0x2000 + i)) for i in range(2)]
    p.close()
    assert fake.calls == ["create", ("rel_free", "before-destroy"), ("rel_free", "before-destroy"), "destroy"]
    keep[0].free()  # already freed by close(): no second call
    assert len(fake.calls) == 4
