"""Pins the CPU oracle (oracle/ifn_oracle.c) before it is trusted as the GPU checker.

Each check is chosen so a plausible oracle bug fails it: a wrong rounding mode
(numpy IEEE binary16), a wrong page/offset split (closed-form and brute-force
slot walks), a wrong GQA head mapping or scale (torch SDPA with enable_gqa), an
off-by-one causal bound (explicit position mask; decode == last prefill row),
a dropped normalisation (closed forms: one key -> V row, equal keys -> mean V).
"""
import math

import numpy as np
import pytest
import torch

import oracle

BS = 16


# ---------------------------------------------------------------- fp16 conversions
def test_half_to_float_exhaustive():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    got = oracle.half_to_float(h)
    ref = h.astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(got.view(np.uint32)[~nan], ref.view(np.uint32)[~nan])
    assert np.isnan(got[nan]).all()


def test_float_to_half_rne_ties_and_ranges():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(1 << 18).astype(np.float32)
         * np.float32(2.0) ** rng.integers(-30, 17, 1 << 18).astype(np.float32))
    h = np.arange(0, 0x7C00, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float64)
    mids = ((h[:-1] + h[1:]) / 2).astype(np.float32)  # exact ties between adjacent halves
    assert np.array_equal(mids.astype(np.float64), (h[:-1] + h[1:]) / 2)
    edge = np.asarray([0.0, -0.0, 65504.0, 65519.996, 65520.0, 1e9, -1e9, 2.0 ** -24, 2.0 ** -25,
                       2.0 ** -25 * 1.0000001, 2.0 ** -26, 6.1e-5, np.inf, -np.inf], np.float32)
    allx = np.concatenate([x, mids, -mids, edge])
    with np.errstate(over="ignore"):
        ref = allx.astype(np.float16)
    got = oracle.float_to_half(allx)
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))


# ---------------------------------------------------------------- slot mapping
def test_slot_mapping_closed_form_and_walk():
    rng = np.random.default_rng(1)
    B, W = 5, 9
    table = rng.permutation(200)[: B * W].astype(np.int32).reshape(B, W)
    seq = rng.integers(0, B, 300).astype(np.int32)
    pos = rng.integers(0, W * BS, 300).astype(np.int32)
    got = oracle.slot_mapping(table, seq, pos, BS)
    assert np.array_equal(got, table[seq, pos // BS] * BS + pos % BS)
    # brute force: enumerate every slot of each row in logical order, then index by position
    walks = [[p * BS + o for p in table[b] for o in range(BS)] for b in range(B)]
    assert got.tolist() == [walks[s][p] for s, p in zip(seq, pos)]
    with pytest.raises(ValueError):
        oracle.slot_mapping(table, seq[:1], np.asarray([W * BS], np.int32), BS)


# ---------------------------------------------------------------- store_kv
def _rand16(rng, *shape):
    return rng.standard_normal(shape, dtype=np.float32).astype(np.float16)


def test_store_kv_equals_dense_scatter_and_spares_other_pages():
    rng = np.random.default_rng(2)
    P, hkv, d, T = 12, 4, 64, 40
    pool = _rand16(rng, 2, P, BS, hkv, d)
    before = pool.copy()
    slots = rng.permutation(P * BS)[:T].astype(np.int32)
    slots[3] = -1              # negative slot: skipped
    slots[7] = P * BS + 5      # beyond the pool: skipped
    active = rng.random(T) > 0.25
    k, v = _rand16(rng, T, hkv, d), _rand16(rng, T, hkv, d)
    oracle.store_kv(pool, slots, active, k, v)
    exp = before.copy()
    flat = exp.reshape(2, P * BS, hkv, d)
    for t in range(T):
        if active[t] and 0 <= slots[t] < P * BS:
            flat[0, slots[t]] = k[t]
            flat[1, slots[t]] = v[t]
    assert np.array_equal(pool.view(np.uint16), exp.view(np.uint16))
    written = {int(s) // BS for t, s in enumerate(slots) if active[t] and 0 <= s < P * BS}
    for p in set(range(P)) - written:  # sentinel pages bit-identical
        assert np.array_equal(pool[:, p].view(np.uint16), before[:, p].view(np.uint16))


def test_paged_store_gather_equals_contiguous_cache():
    """Paged write then block-table gather == the contiguous cache of buffers.py:24-45 (model.py:134-137)."""
    rng = np.random.default_rng(3)
    P, hkv, d, L = 20, 2, 32, 70
    table = rng.permutation(P)[: -(-L // BS)].astype(np.int32)[None]
    pool = np.zeros((2, P, BS, hkv, d), np.float16)
    contiguous = np.zeros((2, L, hkv, d), np.float16)
    k, v = _rand16(rng, L, hkv, d), _rand16(rng, L, hkv, d)
    for start in range(0, L, 17):  # chunked appends
        n = min(17, L - start)
        pos = np.arange(start, start + n, dtype=np.int32)
        sl = oracle.slot_mapping(table, np.zeros(n, np.int32), pos, BS)
        oracle.store_kv(pool, sl, None, k[start:start + n], v[start:start + n])
        contiguous[0, start:start + n], contiguous[1, start:start + n] = k[start:start + n], v[start:start + n]
    gathered = pool[:, table[0]].reshape(2, -1, hkv, d)[:, :L]
    assert np.array_equal(gathered.view(np.uint16), contiguous.view(np.uint16))


# ---------------------------------------------------------------- attention
def _case(rng, B, hq, hkv, d, lens, P=None, tail=False):
    pages = [-(-int(L) // BS) for L in lens]
    P = P or sum(pages) + 3
    W = max(pages)
    perm = rng.permutation(P).astype(np.int32)
    table = np.zeros((B, W), np.int32)
    off = 0
    for b in range(B):
        table[b, :pages[b]] = perm[off:off + pages[b]]
        off += pages[b]
    pool = _rand16(rng, 2, P, BS, hkv, d)
    if tail:
        pool = (pool.astype(np.float32) * np.where(rng.random(pool.shape) < 0.05, 8, 1)).astype(np.float16)
    return pool, table, np.asarray(lens, np.int32)


def _gather(pool, table, b, L):
    kv = pool[:, table[b]].reshape(2, -1, pool.shape[3], pool.shape[4])[:, :L]
    return kv[0], kv[1]  # [L, Hkv, D] each


def _sdpa64(q, k, v, mask=None, scale=None):
    """torch SDPA in float64 on CPU with GQA. q [T,Hq,D], k/v [L,Hkv,D]."""
    tq = torch.from_numpy(q.astype(np.float64)).transpose(0, 1)[None]
    tk = torch.from_numpy(k.astype(np.float64)).transpose(0, 1)[None]
    tv = torch.from_numpy(v.astype(np.float64)).transpose(0, 1)[None]
    m = None if mask is None else torch.from_numpy(mask)
    o = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, attn_mask=m, enable_gqa=True, scale=scale)
    return o[0].transpose(0, 1).numpy()


def _fp16_close(got16, ref64):
    """Within one fp16 ulp of the float64 reference (the oracle rounds once at the end)."""
    g = got16.astype(np.float64)
    ulp = np.maximum(np.abs(ref64), 2.0 ** -14) * 2.0 ** -10
    assert np.all(np.abs(g - ref64) <= ulp + 1e-6), float(np.max(np.abs(g - ref64) / (ulp + 1e-6)))


@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (32, 8, 128), (4, 4, 64), (8, 1, 32)])
def test_decode_matches_torch_sdpa_gqa(hq, hkv, d):
    rng = np.random.default_rng(hq * 100 + hkv + d)
    lens = [1, 15, 16, 17, 100, 257]
    pool, table, sl = _case(rng, len(lens), hq, hkv, d, lens, tail=True)
    q = _rand16(rng, len(lens), hq, d)
    out = oracle.paged_attention(q, pool, table, sl)
    for b, L in enumerate(lens):
        k, v = _gather(pool, table, b, L)
        _fp16_close(out[b], _sdpa64(q[b][None], k, v)[0])


def test_prefill_matches_torch_sdpa_with_position_mask():
    rng = np.random.default_rng(7)
    hq, hkv, d, start, T = 16, 8, 128, 45, 38
    pool, table, _ = _case(rng, 1, hq, hkv, d, [start + T])
    q = _rand16(rng, 1, T, hq, d)
    out = oracle.paged_attention(q, pool, table, np.asarray([start + T], np.int32))
    k, v = _gather(pool, table, 0, start + T)
    key_pos = np.arange(start + T)
    query_pos = np.arange(start, start + T)
    mask = key_pos[None, :] <= query_pos[:, None]  # model.py:128-132
    _fp16_close(out[0], _sdpa64(q[0], k, v, mask=mask))


def test_float64_brute_force_tiny():
    rng = np.random.default_rng(8)
    hq, hkv, d, L = 4, 2, 8, 21
    pool, table, sl = _case(rng, 1, hq, hkv, d, [L])
    q = _rand16(rng, 1, hq, d)
    scale = 0.37
    out = oracle.paged_attention(q, pool, table, sl, scale=scale)
    k, v = _gather(pool, table, 0, L)
    for h in range(hq):
        g = h // (hq // hkv)
        s = [scale * sum(float(q[0, h, i]) * float(k[j, g, i]) for i in range(d)) for j in range(L)]
        mx = max(s)
        w = [math.exp(x - mx) for x in s]
        ref = np.asarray([sum(w[j] * float(v[j, g, i]) for j in range(L)) / sum(w) for i in range(d)])
        _fp16_close(out[0, h], ref)


def test_closed_forms():
    rng = np.random.default_rng(9)
    hq, hkv, d = 4, 2, 64
    # one key: the output is exactly the V row (p = 1)
    pool, table, sl = _case(rng, 1, hq, hkv, d, [1])
    q = _rand16(rng, 1, hq, d)
    out = oracle.paged_attention(q, pool, table, sl)
    k, v = _gather(pool, table, 0, 1)
    for h in range(hq):
        assert np.array_equal(out[0, h].view(np.uint16), v[0, h // 2].view(np.uint16))
    # all keys equal: uniform weights -> mean of V
    L = 40
    pool, table, sl = _case(rng, 1, hq, hkv, d, [L])
    kv = pool[:, table[0]].reshape(2, -1, hkv, d)
    kv[0, :] = kv[0, 0]
    pool[:, table[0]] = kv.reshape(2, -1, BS, hkv, d)
    out = oracle.paged_attention(q, pool, table, sl)
    _, v = _gather(pool, table, 0, L)
    for h in range(hq):
        _fp16_close(out[0, h], v[:, h // 2].astype(np.float64).mean(0))
    # one dominant logit selects its V row
    pool, table, sl = _case(rng, 1, 2, 1, d, [33])
    qq = np.zeros((1, 2, d), np.float16)
    qq[0, :, 0] = 1.0
    kv = pool[:, table[0]].reshape(2, -1, 1, d)
    kv[0, :, 0, 0] = 0.0
    kv[0, 20, 0, 0] = 2000.0
    pool[:, table[0]] = kv.reshape(2, -1, BS, 1, d)
    out = oracle.paged_attention(qq, pool, table, sl)
    assert np.array_equal(out[0, 0].view(np.uint16), kv[1, 20, 0].view(np.uint16))


def test_invariant_to_physical_page_order_and_chunking():
    rng = np.random.default_rng(10)
    hq, hkv, d, L = 16, 8, 128, 150
    pool, table, sl = _case(rng, 1, hq, hkv, d, [L])
    q = _rand16(rng, 1, L, hq, d)
    full = oracle.paged_attention(q, pool, table, sl)
    # relabel physical pages: same logical content, different ids
    perm = rng.permutation(pool.shape[1])
    pool2 = np.empty_like(pool)
    pool2[:, perm] = pool
    table2 = perm[table].astype(np.int32)
    assert np.array_equal(oracle.paged_attention(q, pool2, table2, sl).view(np.uint16), full.view(np.uint16))
    # chunked prefill == unchunked (reference tests/test_cached_forward.py:107-117)
    parts = [oracle.paged_attention(q[:, s:e], pool, table, np.asarray([e], np.int32))
             for s, e in [(0, 50), (50, 51), (51, 150)]]
    assert np.array_equal(np.concatenate(parts, 1).view(np.uint16), full.view(np.uint16))
    # decode at position L-1 == last row of the causal prefill
    dec = oracle.paged_attention(q[:, -1], pool, table, sl)
    assert np.array_equal(dec.view(np.uint16), full[:, -1].view(np.uint16))


def test_inactive_rows_untouched_and_bad_tables_rejected():
    rng = np.random.default_rng(11)
    pool, table, sl = _case(rng, 3, 4, 2, 32, [5, 9, 30])
    q = _rand16(rng, 3, 4, 32)
    prior = _rand16(rng, 3, 4, 32)
    out = oracle.paged_attention(q, pool, table, sl, active_mask=np.asarray([1, 0, 1], bool), out=prior)
    assert np.array_equal(out[1].view(np.uint16), prior[1].view(np.uint16))
    bad = table.copy()
    bad[0, 0] = pool.shape[1]
    with pytest.raises(ValueError):
        oracle.paged_attention(q, pool, bad, sl)


# ---------------- pre-append step: q/k RMSNorm + rotary, k/v cast + store ----------------

def _rope64(max_pos, d, base):
    inv = 1.0 / (base ** (np.arange(0, d, 2, dtype=np.float64) / d))
    ang = np.arange(max_pos, dtype=np.float64)[:, None] * inv[None, :]
    return np.concatenate([np.cos(ang), np.sin(ang)], axis=1)


def _prep64(x, w, rope_row, eps):
    """float64 restatement: x * rsqrt(mean(x^2) + eps) * w, then (x1 c - x2 s, x2 c + x1 s)."""
    x = x.astype(np.float64)
    y = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w.astype(np.float64)
    h = x.shape[-1] // 2
    c, s = rope_row[:h], rope_row[h:]
    return np.concatenate([y[..., :h] * c - y[..., h:] * s, y[..., h:] * c + y[..., :h] * s], axis=-1)


def _prep_case(rng, T=5, hq=4, hkv=2, d=64, P=6, bs=16, max_pos=300):
    q = rng.standard_normal((T, hq, d)).astype(np.float32) * 3
    k = rng.standard_normal((T, hkv, d)).astype(np.float32)
    v = rng.standard_normal((T, hkv, d)).astype(np.float32)
    qw = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    kw = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    rope = _rope64(max_pos, d, 1e6).astype(np.float32)
    pos = rng.integers(0, max_pos, T).astype(np.int32)
    slots = rng.permutation(P * bs)[:T].astype(np.int32)
    pool = rng.standard_normal((2, P, bs, hkv, d)).astype(np.float16)
    return q, k, v, qw, kw, rope, pos, slots, pool


def _ulps(a16, b64):
    """|a - b| in units of the fp16 spacing at b (a correctly rounded fp16 of b is within 0.5)."""
    b = np.asarray(b64, np.float64)
    ulp = np.spacing(np.abs(b).astype(np.float16)).astype(np.float64)
    return np.abs(a16.astype(np.float64) - b) / np.maximum(ulp, 2.0 ** -24)


def test_prep_matches_float64_restatement():
    rng = np.random.default_rng(40)
    q, k, v, qw, kw, rope, pos, slots, pool = _prep_case(rng)
    before = pool.copy()
    qo = oracle.qk_norm_rope_append(q, k, v, qw, kw, rope, pos, slots, None, pool, eps=1e-6)
    rope64 = rope.astype(np.float64)
    for t in range(q.shape[0]):
        ref_q = _prep64(q[t], qw, rope64[pos[t]], 1e-6)
        assert _ulps(qo[t], ref_q).max() <= 1.0
        s = slots[t]
        kk = pool[0, s // 16, s % 16]
        assert _ulps(kk, _prep64(k[t], kw, rope64[pos[t]], 1e-6)).max() <= 1.0
        assert np.array_equal(pool[1, s // 16, s % 16].view(np.uint16), v[t].astype(np.float16).view(np.uint16))
    untouched = np.ones(pool.shape[1] * 16, bool)
    untouched[slots] = False
    flat_b, flat_a = before.reshape(2, -1, *before.shape[3:]), pool.reshape(2, -1, *pool.shape[3:])
    assert np.array_equal(flat_b[:, untouched].view(np.uint16), flat_a[:, untouched].view(np.uint16))


def test_prep_rotation_invariants():
    rng = np.random.default_rng(41)
    q, k, v, qw, kw, rope, pos, slots, pool = _prep_case(rng, T=3, d=128)
    ones = np.ones_like(qw)
    # position 0 is the identity rotation: output = x / rms(x) (weights 1)
    pos0 = np.zeros_like(pos)
    q0 = oracle.qk_norm_rope_append(q, k, v, ones, ones, rope, pos0, slots, None, pool.copy(), eps=0.0)
    rms = np.sqrt(np.mean(q.astype(np.float64) ** 2, axis=-1, keepdims=True))
    assert _ulps(q0, q / rms).max() <= 1.0
    # a rotation keeps every (i, i + D/2) pair's norm
    qp = oracle.qk_norm_rope_append(q, k, v, ones, ones, rope, pos, slots, None, pool.copy(), eps=0.0)
    h = q.shape[-1] // 2
    n0 = q0[..., :h].astype(np.float64) ** 2 + q0[..., h:].astype(np.float64) ** 2
    n1 = qp[..., :h].astype(np.float64) ** 2 + qp[..., h:].astype(np.float64) ** 2
    assert np.allclose(n0, n1, rtol=4e-3, atol=1e-4)


def test_prep_rotation_direction_closed_form():
    """Unit vectors pin the rotation's direction (model.py:24-27: (x1 c - x2 s, x2 c + x1 s)):
    e_i -> sqrt(D) (cos t_i at i, sin t_i at i + D/2) and e_{i+D/2} -> sqrt(D) (-sin t_i, cos t_i).
    A transposed sign (x1 c + x2 s) or swapped halves fails."""
    d, h = 64, 32
    rope = _rope64(100, d, 1e4).astype(np.float32)
    ones = np.ones(d, np.float32)
    for i, p in ((0, 7), (5, 33), (31, 99)):
        q = np.zeros((2, 1, d), np.float32)
        q[0, 0, i] = 1.0
        q[1, 0, h + i] = 1.0
        k = np.zeros((2, 1, d), np.float32)
        pool = np.zeros((2, 1, 16, 1, d), np.float16)
        out = oracle.qk_norm_rope_append(q, k, k, ones, ones, rope, np.full(2, p, np.int32),
                                         np.asarray([-1, -1], np.int32), None, pool, eps=0.0).astype(np.float64)
        c, s_ = float(rope[p, i]), float(rope[p, h + i])
        r = math.sqrt(d)
        exp0 = np.zeros(d); exp0[i], exp0[h + i] = r * c, r * s_
        exp1 = np.zeros(d); exp1[i], exp1[h + i] = -r * s_, r * c
        assert np.allclose(out[0, 0], exp0, atol=r * 2e-3), (i, p)
        assert np.allclose(out[1, 0], exp1, atol=r * 2e-3), (i, p)


def test_rope_table_follows_the_reference_float32_order():
    """rope_table against an independent float32 restatement of _precompute_rope (model.py:18-22)
    in torch float32 ops, step by step, and against closed forms.

    * inverse frequencies 1 / base^(2i/D): within 2 float32 ulps (float32 pow is
      implementation-defined: numpy and torch differ by up to 2 ulps here);
    * angles: the float32 products p * f_i of the table's own frequencies, exactly;
    * cos / sin of those angles: within 2 float32 ulps of torch's float32 cos / sin;
    * row 0 is [1 .. 1 | 0 .. 0]; column 0 has frequency 1 exactly, so it is cos(p) / sin(p) of the
      exact integer p; the slowest column turns by base^(-(D-2)/D) per position (a table built on
      arange(0, D) / D, on i / D or with the halves swapped fails one of these)."""
    from infurnace_amd.kernels import rope_table
    for d, base, n in ((128, 1e6, 40960), (64, 1e4, 4096)):
        tab = rope_table(n, d, base).numpy().astype(np.float64)
        h = d // 2
        inv_t = (1.0 / (torch.tensor(base, dtype=torch.float32) **
                        (torch.arange(0, d, 2, dtype=torch.float32) / d))).numpy()
        # the table's frequencies, recovered from row 1 (angle = f_i exactly at p = 1)
        f_tab = np.arctan2(tab[1, h:], tab[1, :h])
        assert np.all(np.abs(f_tab - inv_t) <= 3 * np.spacing(inv_t.astype(np.float32)) + 1e-7 * inv_t)
        f32 = np.float32
        inv = (f32(1) / np.power(f32(base), (np.arange(0, d, 2, dtype=f32) / f32(d)).astype(f32)).astype(f32))
        inv = inv.astype(f32)
        assert np.all(np.abs(inv.view(np.int32).astype(np.int64) - inv_t.view(np.int32).astype(np.int64)) <= 2)
        ang = torch.arange(n, dtype=torch.float32)[:, None] * torch.from_numpy(inv)[None, :]
        ref = torch.cat([ang.cos(), ang.sin()], dim=1).numpy()
        ulps = np.abs(tab.astype(np.float32).view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
        assert ulps.max() <= 2, ulps.max()
        assert np.array_equal(tab[0], np.concatenate([np.ones(h), np.zeros(h)]))
        p = np.arange(n, dtype=np.float64)
        assert np.array_equal(tab[:, 0], np.cos(p).astype(np.float32).astype(np.float64))
        assert np.array_equal(tab[:, h], np.sin(p).astype(np.float32).astype(np.float64))
        f_last = base ** (-(d - 2) / d)
        assert abs(f_tab[-1] - f_last) <= 1e-6 * f_last


def test_fp16_query_deviation_from_fp32_reference():
    """The paged path takes fp16 queries and reads a chunk's own keys back from the fp16 pool; the
    reference attends an fp32 query and, in a prefill chunk, its own fp32 K/V (model.py:105-125,
    183-187).  This measures that deviation on config-1 (decode) and config-3 (prefill chunk)
    shapes against a float64 restatement with the unrounded inputs; it stays inside the fp16
    tolerance (atol 2e-3 / rtol 1e-2) with a large margin."""
    rng = np.random.default_rng(90)
    # config 1: decode, 16 q / 8 kv heads, 512 keys
    pool = rng.standard_normal((2, 32, 16, 8, 128), dtype=np.float32).astype(np.float16)
    table = rng.permutation(32).astype(np.int32)[None]
    q32 = rng.standard_normal((1, 16, 128), dtype=np.float32)
    got = oracle.paged_attention(q32.astype(np.float16), pool, table, np.asarray([512], np.int32)).astype(np.float64)
    kk = pool[0][table[0]].reshape(512, 8, 128).astype(np.float64)
    vv = pool[1][table[0]].reshape(512, 8, 128).astype(np.float64)
    ref = np.zeros((16, 128))
    for h in range(16):
        s = kk[:, h // 2] @ q32[0, h].astype(np.float64) / math.sqrt(128)
        p = np.exp(s - s.max())
        ref[h] = p @ vv[:, h // 2] / p.sum()
    e1 = np.abs(got[0] - ref)
    assert np.all(e1 <= 2e-3 + 1e-2 * np.abs(ref)) and e1.max() < 1e-3, e1.max()
    # config 3 shapes: a 128-query chunk at position 1920 over 2048 keys; its own K/V in fp32
    T, start = 128, 1920
    table = rng.permutation(128).astype(np.int32)[None]
    pool = rng.standard_normal((2, 128, 16, 8, 128), dtype=np.float32).astype(np.float16)
    k32 = rng.standard_normal((T, 8, 128), dtype=np.float32)
    v32 = rng.standard_normal((T, 8, 128), dtype=np.float32)
    slots = oracle.slot_mapping(table, np.zeros(T, np.int32), np.arange(start, start + T, dtype=np.int32))
    oracle.store_kv(pool, slots, None, k32.astype(np.float16), v32.astype(np.float16))
    q32 = rng.standard_normal((T, 16, 128), dtype=np.float32)
    got = oracle.paged_attention(q32.astype(np.float16)[None], pool, table,
                                 np.asarray([start + T], np.int32))[0].astype(np.float64)
    kk = pool[0][table[0]].reshape(2048, 8, 128).astype(np.float64)
    vv = pool[1][table[0]].reshape(2048, 8, 128).astype(np.float64)
    kk[start:], vv[start:] = k32, v32  # the reference attends the chunk's own fp32 K/V
    e3 = 0.0
    for h in range(16):
        s = (q32[:, h].astype(np.float64) @ kk[:, h // 2].T) / math.sqrt(128)
        s[np.triu(np.ones((T, 2048), bool), k=start + 1)] = -np.inf
        p = np.exp(s - s.max(axis=1, keepdims=True))
        ref = (p @ vv[:, h // 2]) / p.sum(axis=1, keepdims=True)
        err = np.abs(got[:, h] - ref)
        assert np.all(err <= 2e-3 + 1e-2 * np.abs(ref)), (h, err.max())
        e3 = max(e3, float(err.max()))
    assert e3 < 1e-3, e3


def test_prep_skips_inactive_bad_slots_and_positions():
    rng = np.random.default_rng(42)
    q, k, v, qw, kw, rope, pos, slots, pool = _prep_case(rng, T=4)
    slots[1] = pool.shape[1] * 16 + 3      # out of range
    pos[2] = rope.shape[0]                 # outside the table
    active = np.array([1, 1, 1, 0], np.uint8)
    before = pool.copy()
    qo = oracle.qk_norm_rope_append(q, k, v, qw, kw, rope, pos, slots, active, pool)
    assert np.all(qo[2] == 0)
    changed = np.nonzero((before.reshape(2, -1, *before.shape[3:]).view(np.uint16) !=
                          pool.reshape(2, -1, *pool.shape[3:]).view(np.uint16)).any(axis=(0, 2, 3)))[0]
    assert set(changed.tolist()) <= {int(slots[0])}
