"""Array carriers at the boundary, on the GPU: callers that hold no torch tensors.

* objects that only export DLPack, or only the CUDA array interface, are taken without a copy
  by every array argument (outputs through ``out=`` land in the caller's memory), with results
  bit-identical to the same call on torch tensors;
* a caller with raw ``hipMalloc`` memory describes it with ``DeviceArray``;
* a caller with no array library at all calls the C ABI through ctypes with plain addresses,
  checked against the oracle.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from gpu_util import assert_attn_close, say, to_dev
from infurnace_amd import _capi
from infurnace_amd.kernels import DeviceArray, paged_attention, store_kv

pytestmark = pytest.mark.gpu


class OnlyDLPack:
    """A foreign array: nothing but the DLPack protocol (over a torch tensor's memory)."""

    def __init__(self, t):
        self._t = t

    def __dlpack__(self, **kw):
        return self._t.__dlpack__(**kw)

    def __dlpack_device__(self):
        return self._t.__dlpack_device__()


class OnlyCAI:
    """A foreign array: nothing but ``__cuda_array_interface__``."""

    def __init__(self, t):
        self._t = t
        self.__cuda_array_interface__ = t.__cuda_array_interface__


def _case(rng, dev):
    lens = np.asarray([37, 300, 1, 129], np.int32)
    pages = -(-lens // 16)
    P = int(pages.sum()) + 3
    perm = rng.permutation(P).astype(np.int32)
    table = np.zeros((4, pages.max()), np.int32)
    off = 0
    for b, n in enumerate(pages):
        table[b, :n] = perm[off:off + n]
        off += n
    pool = rng.standard_normal((2, P, 16, 8, 128), dtype=np.float32).astype(np.float16)
    q = rng.standard_normal((4, 16, 128), dtype=np.float32).astype(np.float16)
    k = rng.standard_normal((4, 8, 128), dtype=np.float32).astype(np.float16)
    v = rng.standard_normal((4, 8, 128), dtype=np.float32).astype(np.float16)
    pos = lens - 1
    slots = (table[np.arange(4), pos // 16] * 16 + pos % 16).astype(np.int32)
    return pool, table, lens, q, k, v, slots


@pytest.mark.parametrize("carrier", [OnlyDLPack, OnlyCAI])
def test_foreign_carriers_match_torch_bit_for_bit(dev, carrier):
    say(f"carrier {carrier.__name__}")
    rng = np.random.default_rng(5)
    pool, table, lens, q, k, v, slots = _case(rng, dev)
    res = []
    for wrap in (lambda t: t, carrier):
        p = to_dev(pool, dev)
        args = [to_dev(x, dev) for x in (table, lens, q, k, v, slots)]
        bt, sl, qd, kd, vd, sd = args
        out = torch.full_like(qd, 3.0)
        store_kv(wrap(p), wrap(sd), None, wrap(kd), wrap(vd))
        paged_attention(wrap(qd), wrap(p), wrap(bt), wrap(sl), None, out=wrap(out))
        torch.cuda.synchronize()
        res.append((out, p))
    (o1, p1), (o2, p2) = res
    assert torch.equal(p1.view(torch.int16), p2.view(torch.int16)), "pools differ"
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16)), "outputs differ"
    host = pool.copy()
    oracle.store_kv(host, slots, None, k, v)
    assert_attn_close(o2, oracle.paged_attention(q, host, table, lens), f"{carrier.__name__} vs oracle")


class Hip:
    """The few HIP runtime calls a caller without torch tensors needs."""

    def __init__(self):
        self.lib = ctypes.CDLL("libamdhip64.so")
        self.lib.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
        self.lib.hipFree.argtypes = [ctypes.c_void_p]
        self.lib.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        self.lib.hipMemset.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t]
        self.ptrs = []

    def upload(self, a: np.ndarray) -> int:
        p = self.alloc(a.nbytes)
        assert self.lib.hipMemcpy(p, a.ctypes.data, a.nbytes, 1) == 0  # hipMemcpyHostToDevice
        return p

    def alloc(self, n: int, zero: bool = False) -> int:
        p = ctypes.c_void_p()
        assert self.lib.hipMalloc(ctypes.byref(p), max(n, 1)) == 0
        self.ptrs.append(p.value)
        if zero:
            assert self.lib.hipMemset(p.value, 0, n) == 0
        return p.value

    def download(self, p: int, like: np.ndarray) -> np.ndarray:
        out = np.empty_like(like)
        assert self.lib.hipDeviceSynchronize() == 0
        assert self.lib.hipMemcpy(out.ctypes.data, p, out.nbytes, 2) == 0  # hipMemcpyDeviceToHost
        return out

    def free(self):
        self.lib.hipDeviceSynchronize()
        for p in self.ptrs:
            self.lib.hipFree(p)
        self.ptrs = []


def test_raw_hip_memory_through_device_array(dev):
    say("carrier DeviceArray over hipMalloc")
    rng = np.random.default_rng(6)
    pool, table, lens, q, k, v, slots = _case(rng, dev)
    hip = Hip()
    try:
        arr = {n: DeviceArray(hip.upload(a), a.shape, a.dtype, device=dev.index or 0)
               for n, a in dict(pool=pool, table=table, lens=lens, q=q, k=k, v=v, slots=slots).items()}
        out_p = hip.alloc(q.nbytes)
        out = DeviceArray(out_p, q.shape, np.float16, device=dev.index or 0)
        store_kv(arr["pool"], arr["slots"], None, arr["k"], arr["v"])
        paged_attention(arr["q"], arr["pool"], arr["table"], arr["lens"], None, out=out)
        got = hip.download(out_p, q)
        pool_after = hip.download(arr["pool"].ptr, pool)
    finally:
        hip.free()
    host = pool.copy()
    oracle.store_kv(host, slots, None, k, v)
    assert np.array_equal(pool_after.view(np.int16), host.view(np.int16)), "store through DeviceArray"
    assert_attn_close(torch.from_numpy(got), oracle.paged_attention(q, host, table, lens), "DeviceArray decode")


def test_c_abi_with_plain_addresses(dev):
    """The C ABI as a non-Python or non-torch caller uses it: addresses, sizes, a null stream."""
    say("carrier C ABI with plain addresses")
    rng = np.random.default_rng(7)
    pool, table, lens, q, k, v, slots = _case(rng, dev)
    L = _capi.lib()
    hip = Hip()
    try:
        B, P, mp = 4, pool.shape[1], table.shape[1]
        d_pool, d_table, d_lens, d_q, d_k, d_v, d_slots = (hip.upload(a) for a in (pool, table, lens, q, k, v, slots))
        d_out = hip.alloc(q.nbytes)
        max_len = int(lens.max())
        nbytes = L.ifn_paged_decode_workspace_bytes(B, 16, 8, 128, 16, max_len)
        d_ws = hip.alloc(nbytes, zero=True)
        assert L.ifn_store_kv(d_pool, P, d_slots, None, d_k, d_v, B, 8, 128, 16, None) == 0
        assert L.ifn_paged_decode(d_out, d_q, d_pool, P, d_table, mp, d_lens, None, B, 16, 8, 128, 16, max_len,
                                  0.0, d_ws, nbytes, None) == 0
        got = hip.download(d_out, q)
        ws_after = hip.download(d_ws, np.zeros(256 << 10, np.uint8))
    finally:
        hip.free()
    host = pool.copy()
    oracle.store_kv(host, slots, None, k, v)
    assert_attn_close(torch.from_numpy(got), oracle.paged_attention(q, host, table, lens), "C ABI decode")
    assert not ws_after.any(), "the workspace's ticket area is left zeroed"
