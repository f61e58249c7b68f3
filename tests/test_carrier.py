"""Array carriers at the Python boundary, on the host: DLPack and raw-memory descriptors.

The kernel wrappers accept any DLPack or CUDA-array-interface object and ``DeviceArray`` (raw
address, shape, dtype, strides, device) as well as torch tensors, without copying.  These checks
use host memory; the device-memory cases are in test_carrier_gpu.py.
"""
import gc

import numpy as np
import pytest
import torch

from infurnace_amd.kernels import DeviceArray, KVStoreError, PagedAttentionError, as_tensor, paged_attention, store_kv


def test_numpy_through_dlpack_shares_memory():
    a = np.arange(24, dtype=np.int32).reshape(4, 6)
    t = as_tensor(a)
    assert t.dtype == torch.int32 and tuple(t.shape) == (4, 6) and t.data_ptr() == a.ctypes.data
    t[2, 3] = -1
    assert a[2, 3] == -1


@pytest.mark.parametrize("dtype", [np.float16, np.float32, np.int32, np.uint8, np.int64, np.bool_])
def test_device_array_describes_raw_memory(dtype):
    a = (np.arange(60) % 7).astype(dtype).reshape(5, 12)
    whole = torch.from_dlpack(DeviceArray(a.ctypes.data, a.shape, a.dtype, device="cpu", owner=a))
    assert whole.data_ptr() == a.ctypes.data
    assert np.array_equal(whole.numpy(), a)
    # a strided view: columns 1, 4, 7, 10 of every row, transposed
    view = DeviceArray(a.ctypes.data + a.itemsize, (4, 5), a.dtype, device="cpu", strides=(3, 12), owner=a)
    t = torch.from_dlpack(view)
    assert tuple(t.stride()) == (3, 12)
    assert np.array_equal(t.numpy(), a[:, 1::3].T)


def test_device_array_keeps_its_owner_alive():
    a = np.full(1000, 3.5, np.float32)
    t = torch.from_dlpack(DeviceArray(a.ctypes.data, (1000,), np.float32, device="cpu", owner=a))
    del a
    gc.collect()
    assert float(t.sum()) == 3500.0


def test_other_arguments_pass_through_unchanged():
    for x in (None, 3, 2.5, "x", (1, 2), [1], torch.device("cpu")):
        assert as_tensor(x) is x
    t = torch.zeros(3)
    assert as_tensor(t) is t


def test_wrappers_apply_their_own_checks_to_carriers():
    pool = np.zeros((2, 4, 16, 8, 128), np.float16)
    k = np.zeros((1, 8, 128), np.float16)
    with pytest.raises(KVStoreError, match="GPU"):
        store_kv(pool, np.zeros(1, np.int32), None, k, k)
    with pytest.raises(PagedAttentionError):
        paged_attention(np.zeros((1, 16, 128), np.float16), pool, np.zeros((1, 4), np.int32),
                        np.ones(1, np.int32), None)
    assert store_kv.__name__ == "store_kv" and "Append" in store_kv.__doc__


def test_device_array_rejects_bad_descriptions():
    with pytest.raises(ValueError):
        DeviceArray(0, (2, 3), np.float16, strides=(1,))
    with pytest.raises(TypeError):
        torch.from_dlpack(DeviceArray(np.zeros(2).ctypes.data, (2,), np.complex64, device="cpu"))
