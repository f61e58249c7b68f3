"""C-ABI boundary checks that need no GPU: the library loads, exports every
symbol include/infurnace_amd.h declares, and rejects bad arguments on the host
(before any HIP call) with the documented status codes."""
import ctypes
import os
import re

import pytest

from infurnace_amd import _capi

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "infurnace_amd.h")
A = 0x10000  # a 16-byte-aligned fake device address; never dereferenced (validation fails first)


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ifn_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    syms = declared_symbols()
    assert syms == sorted(_capi.SIGNATURES), (syms, sorted(_capi.SIGNATURES))


def test_library_exports_every_declared_symbol():
    lib = _capi.lib()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert lib.ifn_abi_version() == _capi.ABI_VERSION


def test_status_strings():
    for code in (0, -1, -2, -3, -4, -5):
        assert _capi.status_string(code) != "unknown status"
    assert _capi.status_string(-99) == "unknown status"


def test_store_kv_host_validation():
    L = _capi.lib()
    ok = dict(pool=A, P=64, slots=A, mask=None, k=A, v=A, T=4, hkv=8, d=128, bs=16)

    def call(**kw):
        a = {**ok, **kw}
        return L.ifn_store_kv(a["pool"], a["P"], a["slots"], a["mask"], a["k"], a["v"], a["T"], a["hkv"],
                              a["d"], a["bs"], None)

    assert call(pool=None) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert call(slots=None) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert call(P=0) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert call(T=-1) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert call(d=12) == _capi.IFN_ERR_UNSUPPORTED
    assert call(k=A + 8) == _capi.IFN_ERR_ALIGNMENT
    assert call(pool=A + 2) == _capi.IFN_ERR_ALIGNMENT
    assert call(T=0) == _capi.IFN_OK  # nothing to launch
    assert L.ifn_store_kv_layers(A, 0, 64, A, None, A, A, 4, 8, 128, 16, None) == _capi.IFN_ERR_INVALID_ARGUMENT


def test_paged_decode_host_validation():
    L = _capi.lib()
    base = dict(out=A, q=A, pool=A, P=1024, bt=A, W=256, sl=A, am=None, B=32, hq=16, hkv=8, d=128, bs=16,
                msl=4096, scale=0.0, ws=None, wsb=0)

    def call(**kw):
        a = {**base, **kw}
        return L.ifn_paged_decode(a["out"], a["q"], a["pool"], a["P"], a["bt"], a["W"], a["sl"], a["am"], a["B"],
                                  a["hq"], a["hkv"], a["d"], a["bs"], a["msl"], a["scale"], a["ws"], a["wsb"], None)

    assert call(out=None) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert call(hq=12, hkv=8) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert call(bs=24) == _capi.IFN_ERR_UNSUPPORTED  # page sizes compiled: 16, and 32 / 64 for Qwen3 shapes
    assert call(bs=32, hq=8, hkv=8) == _capi.IFN_ERR_UNSUPPORTED  # group 1 has 16-token pages only
    assert call(hq=24) == _capi.IFN_ERR_UNSUPPORTED  # group 3 not compiled
    assert call(d=96) == _capi.IFN_ERR_UNSUPPORTED
    assert call(q=A + 4) == _capi.IFN_ERR_ALIGNMENT
    assert call() == _capi.IFN_ERR_WORKSPACE  # multi-partition launch without a workspace
    need = L.ifn_paged_decode_workspace_bytes(32, 16, 8, 128, 16, 4096)
    assert call(ws=A, wsb=need - 1) == _capi.IFN_ERR_WORKSPACE
    assert call(B=0) == _capi.IFN_OK
    assert call(B=21504) == _capi.IFN_ERR_UNSUPPORTED  # batch beyond the LDS prefix table


def test_fused_append_decode_host_validation():
    L = _capi.lib()
    base = dict(out=A, q=A, pool=A, P=1024, bt=A, W=256, sl=A, am=None, sm=A, nk=A, nv=A, B=32, hq=16, hkv=8,
                d=128, bs=16, msl=4096, scale=0.0, ws=None, wsb=0)

    def call(**kw):
        a = {**base, **kw}
        return L.ifn_paged_decode_append(a["out"], a["q"], a["pool"], a["P"], a["bt"], a["W"], a["sl"], a["am"],
                                         a["sm"], a["nk"], a["nv"], a["B"], a["hq"], a["hkv"], a["d"], a["bs"],
                                         a["msl"], a["scale"], a["ws"], a["wsb"], None)

    assert call(sm=None) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert call(nk=None) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert call(pool=None) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert call(nv=A + 8) == _capi.IFN_ERR_ALIGNMENT
    assert call(hq=24) == _capi.IFN_ERR_UNSUPPORTED
    assert call(B=0) == _capi.IFN_OK
    assert call() == _capi.IFN_ERR_WORKSPACE  # the same workspace rule as ifn_paged_decode


def test_fused_append_prefill_host_validation():
    L = _capi.lib()
    base = dict(out=A, q=A, pool=A, P=1024, bt=A, W=256, qs=0, T=512, nk=A, nv=A, hq=16, hkv=8, d=128, bs=16,
                scale=0.0, ws=None, wsb=0)

    def call(**kw):
        a = {**base, **kw}
        return L.ifn_paged_prefill_append(a["out"], a["q"], a["pool"], a["P"], a["bt"], a["W"], a["qs"], a["T"],
                                          a["nk"], a["nv"], a["hq"], a["hkv"], a["d"], a["bs"], a["scale"], a["ws"],
                                          a["wsb"], None)

    assert call(nk=None) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert call(pool=None) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert call(nv=A + 8) == _capi.IFN_ERR_ALIGNMENT
    assert call(d=256) == _capi.IFN_ERR_UNSUPPORTED
    assert call(T=0) == _capi.IFN_OK
    assert call(qs=4000, T=200) == _capi.IFN_ERR_INVALID_ARGUMENT  # keys past the table


def test_shared_prefix_decode_host_validation():
    L = _capi.lib()
    base = dict(out=A, q=A, pool=A, P=1024, pp=A, S=8, bt=A, W=256, sl=A, am=None, B=32, hq=32, hkv=8, d=128,
                bs=16, msl=4096, scale=0.0, ws=None, wsb=0)

    def call(**kw):
        a = {**base, **kw}
        return L.ifn_paged_decode_shared_prefix(a["out"], a["q"], a["pool"], a["P"], a["pp"], a["S"], a["bt"], a["W"],
                                                a["sl"], a["am"], a["B"], a["hq"], a["hkv"], a["d"], a["bs"], a["msl"],
                                                a["scale"], a["ws"], a["wsb"], None)

    assert call(pp=None) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert call(out=None) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert call(S=-1) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert call(S=257) == _capi.IFN_ERR_INVALID_ARGUMENT  # more shared pages than table columns
    assert call(hq=12, hkv=8) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert call(bs=24) == _capi.IFN_ERR_UNSUPPORTED  # page sizes compiled: 16, and 32 / 64 for Qwen3 shapes
    assert call(bs=32, hq=8, hkv=8) == _capi.IFN_ERR_UNSUPPORTED  # group 1 has 16-token pages only
    assert call(d=256, hq=16) == _capi.IFN_ERR_UNSUPPORTED  # the prefix pass (MFMA) covers D 64 and 128
    assert call(q=A + 4) == _capi.IFN_ERR_ALIGNMENT
    assert call(B=0) == _capi.IFN_OK
    # shared_pages == 0 is the plain decode entry point (same checks and codes)
    assert call(S=0, pp=None) == _capi.IFN_ERR_WORKSPACE
    sizes = [L.ifn_paged_decode_shared_prefix_workspace_bytes(64, 32, 8, 128, 16, s) for s in (0, 8, 256)]
    plain = L.ifn_paged_decode_workspace_bytes(64, 32, 8, 128, 16, 4608)
    assert all(x > plain for x in sizes) and all(x % 256 == 0 for x in sizes)
    assert L.ifn_paged_decode_shared_prefix_workspace_bytes(0, 32, 8, 128, 16, 8) == 0


def test_workspace_sizes():
    L = _capi.lib()
    small = L.ifn_paged_decode_workspace_bytes(1, 16, 8, 128, 16, 512)
    big = L.ifn_paged_decode_workspace_bytes(256, 16, 8, 128, 16, 8192)
    assert 0 < small < big and big % 256 == 0
    assert L.ifn_paged_decode_workspace_bytes(0, 16, 8, 128, 16, 512) == 0
    # partial slots: one per (row, kv head) and per wave of the launch, G x (128 + 2) floats each
    assert big >= (256 * 8 + 2048) * 2 * 130 * 4  # one slot per (row, kv head) and per wave (256 CUs x 8)
    assert L.ifn_paged_prefill_workspace_bytes(512, 1536, 16, 8, 128, 16) > 0


def test_python_wrappers_reject_host_tensors():
    torch = pytest.importorskip("torch")
    from infurnace_amd.kernels import KVStoreError, PagedAttentionError, paged_attention, store_kv
    pool = torch.zeros(2, 4, 16, 8, 128, dtype=torch.float16)
    k = torch.zeros(1, 8, 128, dtype=torch.float16)
    with pytest.raises(KVStoreError):
        store_kv(pool, torch.zeros(1, dtype=torch.int32), None, k, k)
    with pytest.raises(PagedAttentionError):
        paged_attention(torch.zeros(1, 16, 128, dtype=torch.float16), pool, torch.zeros(1, 4, dtype=torch.int32),
                        torch.ones(1, dtype=torch.int32), None)
    with pytest.raises(KVStoreError):
        store_kv(pool.float(), torch.zeros(1, dtype=torch.int32), None, k, k)


def test_prep_and_page_ops_host_validation():
    L = _capi.lib()
    base = dict(qo=A, q=A, k=A, v=A, qw=A, kw=A, rope=A, mp=4096, pos=A, sm=A, am=None, pool=A, P=64, T=4,
                hq=16, hkv=8, d=128, bs=16, eps=1e-6)

    def call(**kw):
        a = {**base, **kw}
        return L.ifn_qk_norm_rope_append(a["qo"], a["q"], a["k"], a["v"], a["qw"], a["kw"], a["rope"], a["mp"],
                                         a["pos"], a["sm"], a["am"], a["pool"], a["P"], a["T"], a["hq"], a["hkv"],
                                         a["d"], a["bs"], a["eps"], None)

    assert call(q=None) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert call(rope=None) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert call(hq=12) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert call(d=127) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert call(eps=-1.0) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert call(eps=float("nan")) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert call(d=512) == _capi.IFN_ERR_UNSUPPORTED
    assert call(T=0) == _capi.IFN_OK
    assert L.ifn_zero_pages(None, 2, 64, A, 3, 8, 128, 16, None) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert L.ifn_zero_pages(A, 0, 64, A, 3, 8, 128, 16, None) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert L.ifn_zero_pages(A + 8, 2, 64, A, 3, 8, 128, 16, None) == _capi.IFN_ERR_ALIGNMENT
    assert L.ifn_zero_pages(A, 2, 64, A, 0, 8, 128, 16, None) == _capi.IFN_OK
    assert L.ifn_copy_pages(A, 2, 64, None, A, 3, 8, 128, 16, None) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert L.ifn_copy_pages(A, 2, 64, A, A, 0, 8, 128, 16, None) == _capi.IFN_OK


def test_prefill_prep_append_host_validation():
    """ifn_paged_prefill_prep_append rejects bad arguments before any HIP call."""
    L = _capi.lib()
    ok = dict(out=A, q=A, k=A, v=A, wq=A, wk=A, rope=A, maxpos=8192, pool=A, P=256, table=A, mp=64, qs=512, T=512,
              hq=16, hkv=8, d=128, bs=16, eps=1e-6)

    def call(**kw):
        a = {**ok, **kw}
        return L.ifn_paged_prefill_prep_append(a["out"], a["q"], a["k"], a["v"], a["wq"], a["wk"], a["rope"],
                                               a["maxpos"], a["pool"], a["P"], a["table"], a["mp"], a["qs"], a["T"],
                                               a["hq"], a["hkv"], a["d"], a["bs"], a["eps"], 0.0, None, 0, None)

    assert call(q=None) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert call(rope=None) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert call(hq=12) == _capi.IFN_ERR_INVALID_ARGUMENT            # not a multiple of the kv heads
    assert call(eps=-1.0) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert call(bs=32) == _capi.IFN_ERR_UNSUPPORTED
    assert call(d=256) == _capi.IFN_ERR_UNSUPPORTED                 # no prefill kernel for this head dim
    assert call(qs=48) == _capi.IFN_ERR_UNSUPPORTED                 # not a multiple of 32: run the two launches
    assert call(k=A + 4) == _capi.IFN_ERR_ALIGNMENT
    assert call(rope=A + 8) == _capi.IFN_ERR_ALIGNMENT
    assert call(T=0) == _capi.IFN_OK
    assert call(qs=512, T=1024) == _capi.IFN_ERR_INVALID_ARGUMENT   # past the table's 1024 keys
    assert call(maxpos=1000) == _capi.IFN_ERR_INVALID_ARGUMENT      # positions past the rotary table


def test_planning_entries_host_validation():
    """The three planning entries (the step's first decode, which writes the step plan) reject a
    missing plan buffer, and otherwise check what their unplanned forms check, before any HIP call."""
    L = _capi.lib()
    ok = dict(out=A, q=A, pool=A, P=1024, bt=A, W=256, sl=A, am=None, sm=A, nk=A, nv=A, B=32, hq=16, hkv=8,
              d=128, bs=16, msl=4096, plan=A, pb=1 << 20, ws=None, wsb=0)

    def plain(**kw):
        a = {**ok, **kw}
        return L.ifn_paged_decode_planning(a["out"], a["q"], a["pool"], a["P"], a["bt"], a["W"], a["sl"], a["am"],
                                           a["B"], a["hq"], a["hkv"], a["d"], a["bs"], a["msl"], 0.0, a["plan"],
                                           a["pb"], a["ws"], a["wsb"], None)

    def append(**kw):
        a = {**ok, **kw}
        return L.ifn_paged_decode_append_planning(a["out"], a["q"], a["pool"], a["P"], a["bt"], a["W"], a["sl"],
                                                  a["am"], a["sm"], a["nk"], a["nv"], a["B"], a["hq"], a["hkv"],
                                                  a["d"], a["bs"], a["msl"], 0.0, a["plan"], a["pb"], a["ws"],
                                                  a["wsb"], None)

    def prep(**kw):
        a = {**ok, **kw}
        return L.ifn_paged_decode_prep_append_planning(a["out"], A, A, A, A, A, A, 8192, A, a["sm"], a["pool"],
                                                       a["P"], a["bt"], a["W"], a["sl"], a["am"], a["B"], a["hq"],
                                                       a["hkv"], a["d"], a["bs"], a["msl"], 0.0, 1e-6, a["plan"],
                                                       a["pb"], a["ws"], a["wsb"], None)

    for call in (plain, append, prep):
        assert call(plan=None) == _capi.IFN_ERR_INVALID_ARGUMENT, call.__name__
        assert call(out=None) == _capi.IFN_ERR_INVALID_ARGUMENT, call.__name__
        assert call(hq=24) == _capi.IFN_ERR_UNSUPPORTED, call.__name__
        assert call(B=0) == _capi.IFN_OK, call.__name__
        assert call(B=0, plan=None) == _capi.IFN_OK, call.__name__  # nothing to decode, nothing to plan
        assert call() == _capi.IFN_ERR_WORKSPACE, call.__name__
    assert append(sm=None) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert append(pool=None) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert prep(sm=None) == _capi.IFN_ERR_INVALID_ARGUMENT


def test_shared_prefix_plan_host_validation():
    """The shared-prefix plan rejects bad arguments on the host; planned and unplanned entries agree on them."""
    L = _capi.lib()
    ok = dict(plan=A, nb=1 << 20, bt=A, mp=288, sl=A, act=None, sp=256, P=4096, B=64, hq=32, hkv=8, d=128, bs=16,
              msl=4608)

    def plan(**kw):
        a = {**ok, **kw}
        return L.ifn_paged_decode_shared_prefix_plan(a["plan"], a["nb"], a["bt"], a["mp"], a["sl"], a["act"], a["sp"],
                                                     a["P"], a["B"], a["hq"], a["hkv"], a["d"], a["bs"], a["msl"], None)

    assert plan(bt=None) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert plan(sp=-1) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert plan(sp=289) == _capi.IFN_ERR_INVALID_ARGUMENT           # more shared pages than table columns
    assert plan(hq=30) == _capi.IFN_ERR_INVALID_ARGUMENT
    assert plan(bs=32) == _capi.IFN_ERR_UNSUPPORTED
    assert plan(B=0) == _capi.IFN_OK
    assert plan(nb=64) == _capi.IFN_ERR_WORKSPACE                   # buffer smaller than the plan
    assert plan(plan=A + 4) == _capi.IFN_ERR_ALIGNMENT
