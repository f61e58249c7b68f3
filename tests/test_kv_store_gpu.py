"""store_kv on the GPU: bit-exact against the oracle's scatter (docs/roadmap.md:339-344 gate:
indexed stores match dense reference updates across page boundaries without inactive or
aliased dummy writes)."""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import randn16, say, to_dev
from infurnace_amd import workloads
from infurnace_amd.kernels import KVStoreError, store_kv, store_kv_layers

pytestmark = pytest.mark.gpu


def _bits_equal(a: torch.Tensor, b) -> bool:
    b = b if isinstance(b, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(b))
    return torch.equal(a.detach().cpu().view(torch.int16), b.cpu().view(torch.int16))


def test_config1_append_bit_exact(dev):
    say("store_kv config1")
    c = workloads.config1()
    pool = to_dev(c["pool"], dev)
    store_kv(pool, to_dev(c["slot_mapping"], dev), None, to_dev(c["new_k"], dev), to_dev(c["new_v"], dev))
    exp = c["pool"].copy()
    oracle.store_kv(exp, c["slot_mapping"], None, c["new_k"], c["new_v"])
    torch.cuda.synchronize()
    assert _bits_equal(pool, exp)


@pytest.mark.parametrize("hkv,d,T", [(8, 128, 1), (8, 128, 37), (8, 128, 512), (4, 64, 50), (2, 40, 33),
                                     (1, 256, 70)])
@pytest.mark.parametrize("mask_kind", ["none", "bool", "uint8"])
def test_random_append_bit_exact_with_inactive_and_bad_slots(dev, hkv, d, T, mask_kind):
    say(f"store_kv random hkv={hkv} d={d} T={T} mask={mask_kind}")
    rng = np.random.default_rng(T * 7 + d)
    P = max(8, -(-T // 16) + 4)
    pool_np = rng.standard_normal((2, P, 16, hkv, d), dtype=np.float32).astype(np.float16)
    slots = rng.permutation(P * 16)[:T].astype(np.int32)
    if T > 3:
        slots[1] = -1
        slots[2] = P * 16 + 3
    active = rng.random(T) > 0.3 if mask_kind != "none" else None
    k = rng.standard_normal((T, hkv, d), dtype=np.float32).astype(np.float16)
    v = rng.standard_normal((T, hkv, d), dtype=np.float32).astype(np.float16)
    pool = to_dev(pool_np, dev)
    am = None if active is None else to_dev(active.astype(np.uint8) if mask_kind == "uint8" else active, dev)
    store_kv(pool, to_dev(slots, dev), am, to_dev(k, dev), to_dev(v, dev))
    oracle.store_kv(pool_np, slots, active, k, v)
    torch.cuda.synchronize()
    assert _bits_equal(pool, pool_np)


def test_layer_selection_and_batched_layers(dev):
    say("store_kv layers")
    rng = np.random.default_rng(5)
    Lyr, P, T = 3, 40, 300
    full_np = rng.standard_normal((Lyr, 2, P, 16, 8, 128), dtype=np.float32).astype(np.float16)
    slots = rng.permutation(P * 16)[:T].astype(np.int32)
    active = rng.random(T) > 0.1
    k = rng.standard_normal((Lyr, T, 8, 128), dtype=np.float32).astype(np.float16)
    v = rng.standard_normal((Lyr, T, 8, 128), dtype=np.float32).astype(np.float16)
    a = to_dev(full_np, dev)
    b = to_dev(full_np, dev)
    for layer in range(Lyr):
        store_kv(a, to_dev(slots, dev), to_dev(active, dev), to_dev(k[layer], dev), to_dev(v[layer], dev),
                 layer=layer)
    store_kv_layers(b, to_dev(slots, dev), to_dev(active, dev), to_dev(k, dev), to_dev(v, dev))
    for layer in range(Lyr):
        oracle.store_kv(full_np[layer], slots, active, k[layer], v[layer])
    torch.cuda.synchronize()
    assert _bits_equal(a, full_np)
    assert _bits_equal(b, full_np)


def test_batched_28_layer_prefill_append_full_size(dev):
    """Config 3's bandwidth-sized append: 28 layers x 2048 tokens in one launch (property check)."""
    say("store_kv_layers 28x2048")
    w = workloads.config3()
    g = torch.Generator(device=dev).manual_seed(33)
    pool = randn16((28, 2, w.num_pages, 16, 8, 128), g, dev)
    before = pool.clone()
    T = w.prompt_len
    slots_np = (w.block_table.astype(np.int64)[np.arange(T) // 16] * 16 + np.arange(T) % 16).astype(np.int32)
    k = randn16((28, T, 8, 128), g, dev)
    v = randn16((28, T, 8, 128), g, dev)
    slots = to_dev(slots_np, dev)
    store_kv_layers(pool, slots, None, k, v)
    torch.cuda.synchronize()
    flat = pool.view(28, 2, -1, 8, 128)
    idx = slots.long()
    assert torch.equal(flat[:, 0, idx].view(torch.int16), k.view(torch.int16))
    assert torch.equal(flat[:, 1, idx].view(torch.int16), v.view(torch.int16))
    bflat = before.view(28, 2, -1, 8, 128)
    bflat[:, :, idx] = flat[:, :, idx]
    assert torch.equal(before.view(torch.int16), pool.view(torch.int16))  # nothing else changed


def test_config2_decode_append_full_pool(dev):
    say("store_kv config2 full pool")
    w = workloads.config2()
    g = torch.Generator(device=dev).manual_seed(2)
    pool = randn16((2, w.num_pages, 16, 8, 128), g, dev)
    before = pool.clone()
    slots = to_dev(w.append_slots, dev)
    k = randn16((w.batch, 8, 128), g, dev)
    v = randn16((w.batch, 8, 128), g, dev)
    active = torch.ones(w.batch, dtype=torch.bool, device=dev)
    active[5] = False
    store_kv(pool, slots, active, k, v, validate=True)
    torch.cuda.synchronize()
    flat = pool.view(2, -1, 8, 128)
    live = slots.long()[active]
    assert torch.equal(flat[0, live].view(torch.int16), k[active].view(torch.int16))
    assert torch.equal(flat[1, live].view(torch.int16), v[active].view(torch.int16))
    before.view(2, -1, 8, 128)[:, live] = flat[:, live]
    assert torch.equal(before.view(torch.int16), pool.view(torch.int16))  # row 5 wrote nothing


def test_debug_validation_rejects_duplicates(dev):
    pool = torch.zeros(2, 4, 16, 8, 128, dtype=torch.float16, device=dev)
    k = torch.zeros(2, 8, 128, dtype=torch.float16, device=dev)
    with pytest.raises(KVStoreError):
        store_kv(pool, torch.tensor([3, 3], dtype=torch.int32, device=dev), None, k, k, validate=True)
    with pytest.raises(KVStoreError):
        store_kv(pool, torch.tensor([3, 64], dtype=torch.int32, device=dev), None, k, k, validate=True)
    # an inactive duplicate is fine
    store_kv(pool, torch.tensor([3, 3], dtype=torch.int32, device=dev),
             torch.tensor([True, False], device=dev), k, k, validate=True)
