"""PagedKVRunner's pre-append path (``_Step.prep_store_attend``) against the oracle pipeline.

The step runs q/k RMSNorm + rotary, the fp16 cast and the append from fp32 projections, then the
attention (model.py:183-200 for decode, :109-138 for a prefill chunk).  It has three branches:

* a prefill chunk: ``qk_norm_rope_append`` then causal ``paged_attention(query_start=...)``;
* a decode step without a shared prefix: one fused launch (``qk_norm_rope_store_and_decode``);
* a decode step over a shared prefix: ``qk_norm_rope_append`` then the shared-prefix decode.

The reference is the oracle's own pipeline on a host pool the oracle writes: for each step,
``orc_qk_norm_rope_append`` at the runner's slots (from the fp32 projections, not from the GPU's q or
pool), then ``orc_paged_attention`` with the runner's tables.  Attention is compared at atol 2e-3 /
rtol 1e-2; after every step the device pool must equal the oracle's host pool with V bit-exact and
K within one fp16 ulp (the pre-append's q/k bar), every other byte untouched.
"""
from dataclasses import dataclass

import numpy as np
import pytest
import torch

import oracle
from gpu_util import assert_attn_close, say, to_dev
from infurnace_amd.kernels import rope_table
from infurnace_amd.runner import PagedKVRunner

pytestmark = pytest.mark.gpu

L, HQ, HKV, D, NB = 2, 16, 8, 128, 96


@dataclass(frozen=True)
class Plan:  # the DecodePlan fields the runner reads (src/infurnace/scheduler/plan.py:16-28)
    slots: tuple
    positions: tuple
    active_mask: tuple
    block_tables: tuple = ()


class Pipeline:
    """The runner and the oracle side by side: the same projections go to both."""

    def __init__(self, dev, seed, **kw):
        self.dev = dev
        self.rng = np.random.default_rng(seed)
        self.run = PagedKVRunner(L, num_slots=4, max_context=1024, num_kv_heads=HKV, head_dim=D, num_blocks=NB,
                                 device=dev, **kw)
        self.host = np.zeros(tuple(self.run.cache.kv.shape), np.float16)  # the runner's pool starts zeroed
        self.rope = rope_table(2048, D, 1_000_000.0, device=dev)
        self.rope_h = self.rope.cpu().numpy()
        self.qw = (1.0 + 0.1 * self.rng.standard_normal(D)).astype(np.float32)
        self.kw = (1.0 + 0.1 * self.rng.standard_normal(D)).astype(np.float32)
        self.qw_d, self.kw_d = to_dev(self.qw, dev), to_dev(self.kw, dev)

    def proj(self, T):
        f = lambda *s: self.rng.standard_normal(s, dtype=np.float32)
        return f(T, HQ, D), f(T, HKV, D), f(T, HKV, D)

    def layer(self, step, layer, T):
        """One layer of a step through prep_store_attend and through the oracle; returns (gpu, ref)."""
        q, k, v = self.proj(T)
        d = lambda a: to_dev(a, self.dev)
        out = step.prep_store_attend(layer, d(q), d(k), d(v), self.qw_d, self.kw_d, self.rope)
        sm = step.slot_mapping.cpu().numpy()
        pos = step.positions.cpu().numpy()
        act = None if step.active is None else step.active.cpu().numpy()
        q16 = oracle.qk_norm_rope_append(q, k, v, self.qw, self.kw, self.rope_h, pos, sm, act, self.host[layer])
        if step.query_start is not None:  # prefill chunk of one sequence
            table = step.block_tables.cpu().numpy().reshape(1, -1)
            n = step.query_start + T
            ref = oracle.paged_attention(q16[None], self.host[layer], table, np.asarray([n], np.int32))[0]
        else:
            table = step.block_tables.cpu().numpy()
            lens = np.minimum(step.seq_lens.cpu().numpy(), step.max_len).astype(np.int32)
            ref = oracle.paged_attention(q16, self.host[layer], table, lens, act)
        return out, ref

    def check_pool(self, what):
        torch.cuda.synchronize(self.dev)
        got = self.run.cache.kv.cpu().numpy()
        v_ok = np.array_equal(got[:, 1].view(np.uint16), self.host[:, 1].view(np.uint16))
        assert v_ok, f"{what}: V pages differ from the oracle's pool"
        diff = np.abs(got[:, 0].view(np.uint16).astype(np.int32) - self.host[:, 0].view(np.uint16).astype(np.int32))
        assert int(diff.max()) <= 1, f"{what}: K pages differ from the oracle's pool by more than one fp16 ulp"


def test_prep_prefill_chunks_then_fused_decode(dev):
    """Branches 1 and 2: chunked prefill (32-aligned and unaligned starts) and fused decode with a
    padding row, all from fp32 projections."""
    say("runner prep: prefill chunks + fused decode")
    p = Pipeline(dev, 61)
    run = p.run
    for slot, start, T in ((0, 0, 64), (0, 64, 40), (1, 0, 37), (1, 37, 27)):
        step = run.begin_prefill(slot, start, T)
        for l in range(L):
            out, ref = p.layer(step, l, T)
            assert_attn_close(out, ref, f"prep prefill slot {slot} start {start} layer {l}")
        p.check_pool(f"prefill slot {slot} start {start}")
    for it in range(4):
        rows = [(0, True), (2, False), (1, True)]
        plan = Plan(tuple(s for s, _ in rows), tuple(run.length(s) if a else 0 for s, a in rows),
                    tuple(a for _, a in rows))
        step = run.begin_decode(plan)
        assert step.shared_prefix is None  # the fused branch
        for l in range(L):
            out, ref = p.layer(step, l, len(rows))
            for i, (s, a) in enumerate(rows):
                if a:
                    assert_attn_close(out[i:i + 1], ref[i:i + 1], f"prep fused decode {it} slot {s} layer {l}")
        p.check_pool(f"fused decode {it}")


def test_prep_decode_over_shared_prefix(dev):
    """Branch 3: rows attached to one cached prompt decode through the pre-append launch and the
    shared-prefix decode."""
    say("runner prep: decode over a shared prefix")
    p = Pipeline(dev, 62, prefix_namespace=("toy", "fp16"), shared_prefix_min_pages=2)
    run = p.run
    prompt = list(range(900, 900 + 100))  # 6 complete blocks + 4 tokens
    step = run.begin_prefill(0, 0, 100)
    for l in range(L):
        out, ref = p.layer(step, l, 100)
        assert_attn_close(out, ref, f"prep prompt layer {l}")
    run.publish_prefix(0, prompt)
    for s, extra in ((1, 9), (2, 30)):
        n = run.attach_prefix(s, prompt[:96] + list(range(extra)))
        assert n == 96
        step = run.begin_prefill(s, n, extra)
        for l in range(L):
            out, ref = p.layer(step, l, extra)
            assert_attn_close(out, ref, f"prep suffix slot {s} layer {l}")
    p.check_pool("prefix + suffixes")
    for it in range(3):
        rows = [(1, True), (2, True), (0, True)]
        plan = Plan(tuple(s for s, _ in rows), tuple(run.length(s) for s, _ in rows), tuple(a for _, a in rows))
        step = run.begin_decode(plan)
        assert step.shared_prefix is not None and step.shared_prefix.numel() == 6
        for l in range(L):
            out, ref = p.layer(step, l, len(rows))
            assert_attn_close(out, ref, f"prep shared decode {it} layer {l}")
        p.check_pool(f"shared decode {it}")
