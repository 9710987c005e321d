"""Pins the CPU oracle (oracle/paged_attention.py) before it is trusted as the checker.

Every check here is independent of the oracle's own formula: an fp64 token-by-token brute
force, closed-form known answers, torch's scaled_dot_product_attention (a library routine)
on a contiguous layout, invariants of the paged layout (task.md:8-10, 92, 94, 146), and the
committed golden fixtures.  test_planted_mistakes_are_caught shows each check can fail: it
plants a plausible mistake in a copy of the oracle and asserts a check rejects it.
"""

from __future__ import annotations

import hashlib
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from mx_flash_attn_kernel_opt__amd import workloads as W
from oracle import (combine_partials, paged_decode_fp64, paged_decode_reference,
                    split_partials)

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _case(lens, Hq, Hkv, D, P, seed=0, pool_pages=0, max_pages=None, k_scale=1.0):
    spec = W.custom_spec("t", lens, Hq, Hkv, D, P, max_pages=max_pages, pool_pages=pool_pages,
                         k_scale=k_scale)
    return W.make_inputs(spec, seed=seed)


def _ref(inp, **kw):
    return paged_decode_reference(inp.q, inp.k_cache, inp.v_cache, inp.block_table,
                                  inp.seq_lens, inp.scale, **kw)


def _fp64(inp):
    return paged_decode_fp64(inp.q, inp.k_cache, inp.v_cache, inp.block_table, inp.seq_lens,
                             inp.scale)


@pytest.mark.parametrize("lens,Hq,Hkv,D,P", [
    ([1, 5, 17, 33], 8, 2, 64, 16),
    ([16, 31, 64], 32, 8, 128, 16),
    ([3, 64, 65], 28, 4, 64, 64),      # group 7, page 64, tail inside one page
    ([40, 7], 16, 16, 32, 16),         # group 1
    ([50], 16, 1, 64, 32),             # group 16
])
def test_fp32_oracle_matches_fp64_brute_force(lens, Hq, Hkv, D, P):
    inp = _case(lens, Hq, Hkv, D, P, seed=len(lens) + D)
    got = _ref(inp).double().numpy()
    exp = _fp64(inp)
    assert np.abs(got - exp).max() < 2e-6


def test_single_token_returns_the_v_row():
    inp = _case([1, 1, 1], 32, 8, 128, 16, seed=3)
    out = _ref(inp)
    for b in range(3):
        page = int(inp.block_table[b, 0])
        expect = inp.v_cache[page, 0].float().repeat_interleave(4, dim=0)
        assert torch.equal(out[b], expect)


def test_constant_v_gives_the_constant():
    inp = _case([1, 9, 100], 16, 4, 64, 16, seed=4)
    c = torch.randn(4, 64).to(torch.bfloat16)
    inp.v_cache[:] = c
    out = _ref(inp)
    assert torch.allclose(out, c.float().repeat_interleave(4, 0).expand_as(out), atol=1e-6)


def test_zero_query_gives_mean_of_valid_v_rows():
    lens = [5, 33, 70]
    inp = _case(lens, 16, 4, 64, 16, seed=5)
    inp.q.zero_()
    out = _ref(inp)
    P = 16
    for b, L in enumerate(lens):
        rows = []
        for t in range(L):
            rows.append(inp.v_cache[int(inp.block_table[b, t // P]), t % P].float())
        mean = torch.stack(rows).mean(0).repeat_interleave(4, 0)
        assert torch.allclose(out[b], mean, atol=1e-6)


def test_identical_keys_give_mean_of_v():
    lens = [20, 48]
    inp = _case(lens, 8, 2, 32, 16, seed=6)
    inp.k_cache[:] = inp.k_cache[0, 0]
    out = _ref(inp)
    q0 = inp.q.clone().zero_()
    ref0 = paged_decode_reference(q0, inp.k_cache, inp.v_cache, inp.block_table,
                                  inp.seq_lens, inp.scale)
    assert torch.allclose(out, ref0, atol=1e-6)


def test_matches_torch_sdpa_on_contiguous_layout():
    """A contiguous cache (arange table) reduces the operator to plain attention, which torch
    computes with its own scaled_dot_product_attention."""
    torch.manual_seed(0)
    B, Hq, Hkv, D, P, L = 3, 32, 8, 128, 16, 200
    npg = math.ceil(L / P)
    q = torch.randn(B, Hq, D).to(torch.bfloat16)
    k = torch.randn(B * npg, P, Hkv, D).to(torch.bfloat16)
    v = torch.randn(B * npg, P, Hkv, D).to(torch.bfloat16)
    table = torch.arange(B * npg, dtype=torch.int32).view(B, npg)
    lens = torch.tensor([L, 1, 137], dtype=torch.int32)
    out = paged_decode_reference(q, k, v, table, lens, 1 / math.sqrt(D))
    kk = k.view(B, npg * P, Hkv, D).double()
    vv = v.view(B, npg * P, Hkv, D).double()
    for b in range(B):
        n = int(lens[b])
        kb = kk[b, :n].permute(1, 0, 2).repeat_interleave(Hq // Hkv, 0)   # [Hq, n, D]
        vb = vv[b, :n].permute(1, 0, 2).repeat_interleave(Hq // Hkv, 0)
        exp = F.scaled_dot_product_attention(q[b].double()[:, None], kb, vb)[:, 0]
        assert torch.allclose(out[b].double(), exp, atol=1e-5)


def test_page_permutation_invariance():
    inp = _case([100, 250, 31], 32, 8, 64, 16, seed=7, pool_pages=60)
    out = _ref(inp)
    perm = torch.randperm(60, generator=torch.Generator().manual_seed(1))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(60)
    out2 = paged_decode_reference(inp.q, inp.k_cache[perm], inp.v_cache[perm],
                                  inv[inp.block_table.long()].int(), inp.seq_lens, inp.scale)
    assert torch.equal(out, out2)


def test_padding_entries_and_unused_slots_are_ignored():
    P = 16
    lens = [1, 17, 40]
    inp = _case(lens, 16, 4, 64, P, seed=8, pool_pages=40, max_pages=6)
    out = _ref(inp)
    bt = inp.block_table.clone()
    used = {int(bt[b, i]) for b, L in enumerate(lens) for i in range(math.ceil(L / P))}
    unused = [p for p in range(40) if p not in used]
    for b, L in enumerate(lens):
        n = math.ceil(L / P)
        bt[b, n:] = torch.tensor(unused[: 6 - n], dtype=torch.int32)
    k, v = inp.k_cache.clone(), inp.v_cache.clone()
    k[unused] = float("nan")
    v[unused] = float("nan")
    for b, L in enumerate(lens):
        if L % P:
            k[int(bt[b, L // P]), L % P:] = float("nan")
            v[int(bt[b, L // P]), L % P:] = float("nan")
    out2 = paged_decode_reference(inp.q, k, v, bt, inp.seq_lens, inp.scale)
    assert torch.equal(out, out2)


def test_kv_head_mapping_is_h_div_group():
    """Swapping KV heads 0 and 1 in the cache must swap query groups 0 and 1 of the output
    (kv = h // group, task.md:62, 140), and leave the other groups alone."""
    inp = _case([30, 70], 32, 8, 64, 16, seed=9)
    out = _ref(inp)
    k, v = inp.k_cache.clone(), inp.v_cache.clone()
    k[:, :, [0, 1]] = k[:, :, [1, 0]]
    v[:, :, [0, 1]] = v[:, :, [1, 0]]
    q = inp.q.clone()
    q[:, 0:4], q[:, 4:8] = inp.q[:, 4:8].clone(), inp.q[:, 0:4].clone()
    out2 = paged_decode_reference(q, k, v, inp.block_table, inp.seq_lens, inp.scale)
    assert torch.equal(out2[:, 0:4], out[:, 4:8])
    assert torch.equal(out2[:, 4:8], out[:, 0:4])
    assert torch.equal(out2[:, 8:], out[:, 8:])


@pytest.mark.parametrize("tps", [16, 32, 48, 112, 512, 4096])
def test_split_and_lse_combine_equal_the_unsplit_result(tps):
    inp = _case([1, 16, 100, 333, 600], 32, 8, 64, 16, seed=10, k_scale=3.0)
    o, lse, nsv = split_partials(inp.q, inp.k_cache, inp.v_cache, inp.block_table,
                                 inp.seq_lens, tps, inp.scale)
    merged = combine_partials(o, lse, nsv)
    assert np.abs(merged - _fp64(inp)).max() < 1e-10


def test_empty_sequence_gives_zeros():
    inp = _case([0, 5], 8, 2, 32, 16, seed=11, max_pages=2)
    inp.seq_lens[0] = 0
    out = _ref(inp)
    assert torch.count_nonzero(out[0]) == 0


# ---------------------------------------------------------------------------------------
# Planted mistakes (in copies of the oracle, on the CPU) must be caught
# ---------------------------------------------------------------------------------------

def _mutant(kind, q, k_cache, v_cache, block_table, seq_lens, scale):
    B, Hq, D = q.shape
    P, Hkv = k_cache.shape[1], k_cache.shape[2]
    G = Hq // Hkv
    out = torch.zeros(B, Hq, D)
    for b in range(B):
        L = int(seq_lens[b])
        if kind == "off_by_one":
            L = max(L - 1, 1)
        for h in range(Hq):
            kvh = h % Hkv if kind == "head_mod" else h // G
            ts = range(L)
            if kind == "page_transposed":
                rows = [(int(block_table[b, t % block_table.shape[1]]), t // block_table.shape[1])
                        for t in ts]
                rows = [(p, min(o, P - 1)) for p, o in rows]
            else:
                rows = [(int(block_table[b, t // P]), t % P) for t in ts]
            kk = torch.stack([k_cache[p, o, kvh].float() for p, o in rows])
            vv = torch.stack([v_cache[p, o, kvh].float() for p, o in rows])
            s = 1.0 if kind == "no_scale" else scale
            w = torch.softmax(kk @ q[b, h].float() * s, 0)
            out[b, h] = w @ vv
    return out


@pytest.mark.parametrize("kind", ["head_mod", "off_by_one", "no_scale", "page_transposed"])
def test_planted_mistakes_are_caught(kind):
    inp = _case([3, 37, 70], 16, 4, 32, 16, seed=12, pool_pages=20)
    bad = _mutant(kind, inp.q, inp.k_cache, inp.v_cache, inp.block_table, inp.seq_lens,
                  inp.scale)
    exp = _fp64(inp)
    assert np.abs(bad.double().numpy() - exp).max() > 1e-3
    good = _mutant("none", inp.q, inp.k_cache, inp.v_cache, inp.block_table, inp.seq_lens,
                   inp.scale)
    assert np.abs(good.double().numpy() - exp).max() < 2e-6


# ---------------------------------------------------------------------------------------
# Golden fixtures (tests/golden/make_golden.py)
# ---------------------------------------------------------------------------------------

def _sha(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


def load_golden(name: str):
    """Regenerate the fixture's inputs from its recipe and check them against its hashes."""
    z = np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False)
    lens = [int(x) for x in z["seq_lens"]]
    Hq, Hkv, D, P, max_pages, pool, seed = (int(x) for x in z["shape"])
    spec = W.custom_spec(name, lens, Hq, Hkv, D, P, max_pages=max_pages, pool_pages=pool)
    inp = W.make_inputs(spec, seed=seed)
    for key, t in (("q", inp.q), ("k_cache", inp.k_cache), ("v_cache", inp.v_cache),
                   ("block_table", inp.block_table)):
        assert _sha(t) == str(z[f"sha_{key}"]), f"{name}: regenerated {key} differs"
    return inp, torch.from_numpy(z["expected"])


@pytest.mark.parametrize("name", ["task_example", "ragged_g7_p64_d64"])
def test_oracle_matches_golden(name):
    inp, expected = load_golden(name)
    out = _ref(inp)
    assert (out - expected).abs().max().item() < 2e-6


# ---------------------------------------------------------------------------------------
# Multi-token queries (seqlen_q > 1) and the end-aligned causal mask
# ---------------------------------------------------------------------------------------

def _mq_case(lens, Hq, Hkv, D, P, sq, seed=0):
    spec = W.custom_spec("mq", lens, Hq, Hkv, D, P, seqlen_q=sq)
    return W.make_inputs(spec, seed=seed)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("lens,Hq,Hkv,D,P,sq", [
    ([1, 5, 17, 40], 8, 2, 64, 16, 3),      # L < seqlen_q: early causal rows see no key
    ([33, 2], 28, 4, 32, 16, 2),             # group 7
    ([70], 16, 16, 64, 32, 5),               # group 1
])
def test_multi_token_fp32_oracle_matches_fp64_brute_force(lens, Hq, Hkv, D, P, sq, causal):
    inp = _mq_case(lens, Hq, Hkv, D, P, sq, seed=sq + D)
    got = _ref(inp, causal=causal).double().numpy()
    exp = paged_decode_fp64(inp.q, inp.k_cache, inp.v_cache, inp.block_table, inp.seq_lens,
                            inp.scale, causal=causal)
    assert got.shape == tuple(inp.q.shape)
    assert np.abs(got - exp).max() < 2e-6


@pytest.mark.parametrize("causal", [False, True])
def test_multi_token_rows_are_single_token_decodes(causal):
    """Query token i of seqlen_q is a one-token decode of q[:, i] over the first L keys, or
    over the first L - seqlen_q + i + 1 keys with the end-aligned causal mask (zeros when that
    is <= 0), checked against the single-token fp64 brute force pinned above."""
    sq = 4
    inp = _mq_case([2, 9, 16, 47], 16, 4, 64, 16, sq, seed=5)
    out = _ref(inp, causal=causal).double().numpy()
    for i in range(sq):
        lens = inp.seq_lens - (sq - 1 - i) if causal else inp.seq_lens
        single = paged_decode_fp64(inp.q[:, i], inp.k_cache, inp.v_cache, inp.block_table,
                                   lens, inp.scale)
        assert np.abs(out[:, i] - single).max() < 2e-6, i


def test_causal_square_case_matches_torch_sdpa_is_causal():
    """With seqlen_q == L the end-aligned mask is the ordinary lower triangle, which torch's
    scaled_dot_product_attention(is_causal=True) computes itself; the last query row of any
    causal call sees every key (equal to the non-causal row)."""
    torch.manual_seed(3)
    Hq, Hkv, D, P, L = 8, 2, 64, 16, 37
    npg = math.ceil(L / P)
    q = torch.randn(1, L, Hq, D).to(torch.bfloat16)
    k = torch.randn(npg, P, Hkv, D).to(torch.bfloat16)
    v = torch.randn(npg, P, Hkv, D).to(torch.bfloat16)
    table = torch.arange(npg, dtype=torch.int32).view(1, npg)
    lens = torch.tensor([L], dtype=torch.int32)
    out = paged_decode_reference(q, k, v, table, lens, 1 / math.sqrt(D), causal=True)
    kk = k.view(npg * P, Hkv, D)[:L].double().permute(1, 0, 2).repeat_interleave(Hq // Hkv, 0)
    vv = v.view(npg * P, Hkv, D)[:L].double().permute(1, 0, 2).repeat_interleave(Hq // Hkv, 0)
    exp = F.scaled_dot_product_attention(q[0].double().permute(1, 0, 2), kk, vv,
                                         is_causal=True)          # [Hq, L, D]
    assert torch.allclose(out[0].double(), exp.permute(1, 0, 2), atol=1e-5)
    full = paged_decode_reference(q, k, v, table, lens, 1 / math.sqrt(D), causal=False)
    assert torch.equal(out[:, -1], full[:, -1])


def _causal_mutant(kind, inp):
    """Copies of the causal rule with plausible mistakes: the top-left aligned mask (query i
    sees keys t <= i) and an end-aligned mask off by one (t < L - seqlen_q + i)."""
    B, sq, Hq, D = inp.q.shape
    out = torch.zeros(B, sq, Hq, D, dtype=torch.float64)
    for i in range(sq):
        if kind == "top_left":
            lens = torch.clamp(inp.seq_lens, max=i + 1)
        else:
            lens = inp.seq_lens - (sq - i)
        out[:, i] = torch.from_numpy(paged_decode_fp64(inp.q[:, i], inp.k_cache, inp.v_cache,
                                                       inp.block_table, lens, inp.scale))
    return out


@pytest.mark.parametrize("kind", ["top_left", "off_by_one"])
def test_planted_causal_mistakes_are_caught(kind):
    inp = _mq_case([5, 30, 64], 8, 2, 32, 16, 4, seed=9)
    exp = _ref(inp, causal=True).double()
    assert (torch.as_tensor(_causal_mutant(kind, inp)) - exp).abs().max().item() > 1e-3


# ---------------------------------------------------------------------------------------
# Paged K/V append (the producer of the page layout)
# ---------------------------------------------------------------------------------------

def _append_case(lens, S, Hkv=4, D=32, P=16, width=6, seed=0):
    from oracle import paged_kv_append_reference
    g = torch.Generator().manual_seed(seed)
    B = len(lens)
    pool = B * width + 3
    k = torch.randn(pool, P, Hkv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(pool, P, Hkv, D, generator=g).to(torch.bfloat16)
    table = torch.randperm(pool, generator=g)[: B * width].to(torch.int32).view(B, width)
    kn = torch.randn(B, S, Hkv, D, generator=g).to(torch.bfloat16)
    vn = torch.randn(B, S, Hkv, D, generator=g).to(torch.bfloat16)
    lens_t = torch.tensor(lens, dtype=torch.int32)
    k2, v2, flags = paged_kv_append_reference(kn, vn, k, v, table, lens_t)
    return k, v, table, kn, vn, lens_t, k2, v2, flags


def test_append_then_decode_is_attention_over_the_concatenated_keys():
    """Round trip: after appending S tokens, decoding L + S tokens equals plain attention
    (torch SDPA) over [the L old rows; the S new rows], gathered independently."""
    lens = [0, 5, 15, 16, 31, 40]
    S = 3
    k, v, table, kn, vn, lens_t, k2, v2, flags = _append_case(lens, S)
    assert not flags
    Hq, Hkv, D, P = 8, 4, 32, 16
    q = torch.randn(len(lens), Hq, D, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
    out = paged_decode_reference(q, k2, v2, table, lens_t + S, 1 / math.sqrt(D))
    for b, L in enumerate(lens):
        old_k = torch.stack([k[int(table[b, t // P]), t % P] for t in range(L)]) if L else \
            torch.zeros(0, Hkv, D, dtype=torch.bfloat16)
        old_v = torch.stack([v[int(table[b, t // P]), t % P] for t in range(L)]) if L else \
            torch.zeros(0, Hkv, D, dtype=torch.bfloat16)
        kk = torch.cat([old_k, kn[b]]).double().permute(1, 0, 2).repeat_interleave(Hq // Hkv, 0)
        vv = torch.cat([old_v, vn[b]]).double().permute(1, 0, 2).repeat_interleave(Hq // Hkv, 0)
        exp = F.scaled_dot_product_attention(q[b].double()[:, None], kk, vv)[:, 0]
        assert torch.allclose(out[b].double(), exp, atol=1e-5), b


def test_append_touches_only_the_new_slots():
    lens = [7, 0, 30]
    k, v, table, kn, vn, lens_t, k2, v2, flags = _append_case(lens, 4, seed=2)
    changed = (k2 != k).flatten(2).any(-1) | (v2 != v).flatten(2).any(-1)   # [pool, P]
    expect = torch.zeros_like(changed)
    for b, L in enumerate(lens):
        for j in range(4):
            pos = L + j
            expect[int(table[b, pos // 16]), pos % 16] = True
    assert torch.equal(changed, expect)


def test_append_flags_overflow_and_bad_pages():
    from oracle import paged_kv_append_reference
    k, v, table, kn, vn, lens_t, _, _, _ = _append_case([94, 10], 3, seed=4)   # row: 96 slots
    table = table.clone()
    table[1, 0] = 10_000
    k2, v2, flags = paged_kv_append_reference(kn, vn, k, v, table, lens_t)
    assert flags == {"seq_too_long", "bad_page"}
    assert torch.equal(k2[int(table[0, 5]), 14:], kn[0, :2])   # positions 94, 95 written


@pytest.mark.parametrize("kind", ["off_by_one", "page_offset_swapped"])
def test_planted_append_mistakes_are_caught(kind):
    """A mutant append (position L + j - 1, or page/offset computed as pos % width, pos // width)
    fails the round-trip decode check."""
    lens = [5, 20, 33]
    S, P, width = 2, 16, 6
    k, v, table, kn, vn, lens_t, k2, v2, _ = _append_case(lens, S, seed=6)
    km, vm = k.clone(), v.clone()
    for b, L in enumerate(lens):
        for j in range(S):
            pos = L + j - (1 if kind == "off_by_one" else 0)
            page, off = ((int(table[b, pos // P]), pos % P) if kind == "off_by_one"
                         else (int(table[b, pos % width]), min(pos // width, P - 1)))
            km[page, off] = kn[b, j]
            vm[page, off] = vn[b, j]
    q = torch.randn(3, 8, 32, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    good = paged_decode_reference(q, k2, v2, table, lens_t + S)
    bad = paged_decode_reference(q, km, vm, table, lens_t + S)
    assert (good - bad).abs().max().item() > 1e-3


# ---------------------------------------------------------------------------------------
# Sharded decode: one shard's unmerged (o, lse) and the merge of gathered shards
# ---------------------------------------------------------------------------------------

def _shard_partials(inp, num_shards, causal=False):
    from mx_flash_attn_kernel_opt__amd import shard_pages
    from oracle import paged_decode_partial_reference
    sq = inp.q.shape[1] if inp.q.dim() == 4 else 1
    parts = []
    for s, (tab, lens) in enumerate(shard_pages(inp.block_table, inp.seq_lens,
                                                inp.k_cache.shape[1], num_shards, sq)):
        parts.append(paged_decode_partial_reference(
            inp.q, inp.k_cache, inp.v_cache, tab, lens, inp.scale,
            causal=causal and s == num_shards - 1))
    return parts


def test_partial_lse_matches_scipy_logsumexp():
    """lse of one shard is log(sum_t exp(scale q.k_t)) over its keys, computed here token by
    token from the contiguous keys with scipy.special.logsumexp (an independent routine)."""
    from scipy.special import logsumexp
    from oracle import paged_decode_partial_reference
    inp = _case([1, 17, 40], 8, 2, 32, 16, seed=21)
    o, lse = paged_decode_partial_reference(inp.q, inp.k_cache, inp.v_cache, inp.block_table,
                                            inp.seq_lens, inp.scale)
    P = 16
    for b, L in enumerate(inp.seq_lens.tolist()):
        pages = inp.block_table[b, :math.ceil(L / P)].long()
        k = inp.k_cache[pages].reshape(-1, 2, 32)[:L].double().numpy()
        for h in range(8):
            logits = k[:, h // 4] @ inp.q[b, h].double().numpy() * inp.scale
            assert abs(lse[b, h].item() - logsumexp(logits)) < 1e-9
    exp = _fp64(inp)
    assert np.abs(o.numpy() - exp).max() < 1e-9


def test_partial_lse_closed_form_for_a_zero_query():
    """q = 0 makes every logit 0: lse = log(L) exactly and o = mean of the V rows."""
    from oracle import paged_decode_partial_reference
    inp = _case([1, 5, 64], 16, 4, 32, 16, seed=22)
    q0 = torch.zeros_like(inp.q)
    _, lse = paged_decode_partial_reference(q0, inp.k_cache, inp.v_cache, inp.block_table,
                                            inp.seq_lens, inp.scale)
    for b, L in enumerate(inp.seq_lens.tolist()):
        assert torch.allclose(lse[b], torch.full_like(lse[b], math.log(L)), atol=1e-12)


def test_empty_shard_rows_are_zero_with_lse_minus_inf():
    from oracle import paged_decode_partial_reference
    inp = _case([0, 9], 8, 2, 32, 16, seed=23)
    o, lse = paged_decode_partial_reference(inp.q, inp.k_cache, inp.v_cache, inp.block_table,
                                            inp.seq_lens, inp.scale)
    assert torch.all(o[0] == 0) and torch.all(torch.isneginf(lse[0]))
    assert torch.all(torch.isfinite(lse[1]))


@pytest.mark.parametrize("num_shards", [1, 2, 3, 4, 7])
def test_merged_shards_equal_the_unsharded_decode(num_shards):
    """Any page sharding, merged, is the unsharded decode (pinned above against SDPA and the
    fp64 brute force); sequences shorter than num_shards pages leave empty shards."""
    from oracle import lse_merge_reference
    inp = _case([0, 1, 16, 17, 70, 200], 16, 4, 64, 16, seed=24 + num_shards)
    parts = _shard_partials(inp, num_shards)
    got = lse_merge_reference(np.stack([p[0].numpy() for p in parts]),
                              np.stack([p[1].numpy() for p in parts]))
    assert np.abs(got - _fp64(inp)).max() < 1e-9


@pytest.mark.parametrize("num_shards", [2, 4])
def test_causal_multi_token_shards_merge_to_the_causal_decode(num_shards):
    """With the last shard masked on its own length (it holds every key some query token must
    not see) and the others unmasked, the merge equals the end-aligned causal decode, including
    rows that see no key at all (L < seqlen_q)."""
    from oracle import lse_merge_reference
    sq = 5
    inp = _mq_case([2, 4, 19, 33, 90, 161], 8, 2, 32, 16, sq, seed=30 + num_shards)
    parts = _shard_partials(inp, num_shards, causal=True)
    got = lse_merge_reference(np.stack([p[0].numpy() for p in parts]),
                              np.stack([p[1].numpy() for p in parts]))
    exp = paged_decode_fp64(inp.q, inp.k_cache, inp.v_cache, inp.block_table, inp.seq_lens,
                            inp.scale, causal=True)
    assert np.abs(got - exp).max() < 1e-9


def test_shard_pages_covers_every_key_once_with_the_tail_in_the_last_shard():
    from mx_flash_attn_kernel_opt__amd import shard_pages
    P, sq = 16, 6
    inp = _mq_case([0, 1, 5, 16, 21, 47, 48, 300], 8, 2, 32, P, sq, seed=40)
    for n in (1, 2, 3, 5, 8):
        shards = shard_pages(inp.block_table, inp.seq_lens, P, n, sq)
        for b, L in enumerate(inp.seq_lens.tolist()):
            keys = []
            for s, (tab, lens) in enumerate(shards):
                ls = int(lens[b])
                pages = tab[b, :math.ceil(ls / P)].tolist()
                keys += [(pg, off) for pg in pages for off in range(P)][:ls]
                if s < n - 1:   # earlier shards hold only keys every query token sees
                    assert len(keys) <= max(L - sq + 1, 0)
            full = inp.block_table[b, :math.ceil(L / P)].tolist()
            assert keys == [(pg, off) for pg in full for off in range(P)][:L]


def _merge_mutant(kind, o, lse):
    m = lse.max(0)
    if kind == "log2_weights":      # lse read as log2 while it is a natural log
        w = np.exp2(lse - m)
    elif kind == "unweighted":      # partials averaged without their softmax mass
        w = np.isfinite(lse).astype(np.float64)
    else:                           # "sum_not_normalised": weights not divided by their sum
        return (np.exp(lse - m)[..., None] * o).sum(0)
    return (w[..., None] * o).sum(0) / w.sum(0)[..., None]


@pytest.mark.parametrize("kind", ["log2_weights", "unweighted", "sum_not_normalised"])
def test_planted_merge_mistakes_are_caught(kind):
    inp = _case([40, 90, 130], 8, 2, 32, 16, seed=41)
    parts = _shard_partials(inp, 3)
    o = np.stack([p[0].numpy() for p in parts])
    lse = np.stack([p[1].numpy() for p in parts])
    assert np.abs(_merge_mutant(kind, o, lse) - _fp64(inp)).max() > 1e-3


def test_planted_causal_on_every_shard_is_caught():
    """Masking every shard on its own length (instead of only the last) hides keys that the
    earlier shards must show."""
    from oracle import lse_merge_reference, paged_decode_partial_reference
    from mx_flash_attn_kernel_opt__amd import shard_pages
    sq = 4
    inp = _mq_case([40, 90], 8, 2, 32, 16, sq, seed=42)
    parts = [paged_decode_partial_reference(inp.q, inp.k_cache, inp.v_cache, t, l, inp.scale,
                                            causal=True)
             for t, l in shard_pages(inp.block_table, inp.seq_lens, 16, 3, sq)]
    got = lse_merge_reference(np.stack([p[0].numpy() for p in parts]),
                              np.stack([p[1].numpy() for p in parts]))
    exp = paged_decode_fp64(inp.q, inp.k_cache, inp.v_cache, inp.block_table, inp.seq_lens,
                            inp.scale, causal=True)
    assert np.abs(got - exp).max() > 1e-3


@pytest.mark.parametrize("sq,causal", [(1, False), (3, True), (3, False)])
def test_append_and_attend_is_masked_attention_over_the_concatenated_keys(sq, causal):
    """The fused reference (append S new tokens, decode their sq queries over L + S keys) equals
    torch SDPA over [old rows; new rows] with an explicit end-aligned mask: query token i sees
    keys t < L + S - sq + i + 1."""
    from oracle import paged_decode_append_reference
    lens = [0, 4, 15, 16, 40]
    S = 3
    k, v, table, kn, vn, lens_t, k2, v2, flags = _append_case(lens, S, seed=12)
    Hq, Hkv, D, P = 8, 4, 32, 16
    g = torch.Generator().manual_seed(13)
    q = torch.randn(len(lens), sq, Hq, D, generator=g).to(torch.bfloat16)
    out, k3, v3, fl = paged_decode_append_reference(q, kn, vn, k, v, table, lens_t,
                                                    1 / math.sqrt(D), causal=causal)
    assert not fl and torch.equal(k3, k2) and torch.equal(v3, v2)
    for b, L in enumerate(lens):
        old_k = torch.stack([k[int(table[b, t // P]), t % P] for t in range(L)]) if L else \
            torch.zeros(0, Hkv, D, dtype=torch.bfloat16)
        old_v = torch.stack([v[int(table[b, t // P]), t % P] for t in range(L)]) if L else \
            torch.zeros(0, Hkv, D, dtype=torch.bfloat16)
        kk = torch.cat([old_k, kn[b]]).double().permute(1, 0, 2).repeat_interleave(Hq // Hkv, 0)
        vv = torch.cat([old_v, vn[b]]).double().permute(1, 0, 2).repeat_interleave(Hq // Hkv, 0)
        n = L + S
        mask = torch.ones(sq, n, dtype=torch.bool)
        if causal:
            mask = torch.arange(n)[None, :] < (n - sq + torch.arange(sq)[:, None] + 1)
        exp = F.scaled_dot_product_attention(q[b].double().permute(1, 0, 2), kk, vv,
                                             attn_mask=mask)          # [Hq, sq, D]
        assert torch.allclose(out[b].double(), exp.permute(1, 0, 2), atol=1e-5), b


# ------------------------------------------------------------------------------------------
# fp8 (OCP e4m3fn) K/V cache oracle
# ------------------------------------------------------------------------------------------

def test_fp8_dequantize_known_codes():
    """torch's e4m3fn conversion, which the fp8 oracle relies on, on codes whose values the
    OCP format fixes: 0x38 = 1, 0x7e = 448 (largest finite), 0x01 = 2^-9 (smallest subnormal),
    0x08 = 2^-6 (smallest normal), 0x80 = -0, 0x7f = NaN, and the scale multiplies."""
    from oracle import fp8_dequantize
    codes = torch.tensor([0x38, 0x7E, 0x01, 0x08, 0x80, 0x7F, 0xB8, 0x3C], dtype=torch.uint8)
    x = fp8_dequantize(codes.view(torch.float8_e4m3fn), 1.0)
    assert x[0] == 1.0 and x[1] == 448.0 and x[2] == 2.0 ** -9 and x[3] == 2.0 ** -6
    assert x[4] == 0.0 and math.copysign(1.0, x[4].item()) == -1.0
    assert torch.isnan(x[5]) and x[6] == -1.0 and x[7] == 1.5
    assert torch.equal(fp8_dequantize(codes[:4].view(torch.float8_e4m3fn), 0.25), x[:4] * 0.25)


def _fp8_case(seed, lens, Hq=8, Hkv=2, D=64, P=16):
    g = torch.Generator().manual_seed(seed)
    B = len(lens)
    width = max(1, -(-max(lens) // P))
    pool = B * width + 3
    k8 = (torch.randn(pool, P, Hkv, D, generator=g) * 3).to(torch.float8_e4m3fn)
    v8 = (torch.randn(pool, P, Hkv, D, generator=g) * 3).to(torch.float8_e4m3fn)
    q = torch.randn(B, Hq, D, generator=g).to(torch.bfloat16)
    table = torch.randperm(pool, generator=g)[: B * width].to(torch.int32).view(B, width)
    return q, k8, v8, table, torch.tensor(lens, dtype=torch.int32)


def test_fp8_oracle_equals_the_bf16_oracle_on_the_same_values():
    """Every e4m3fn value is a bf16 value, so the fp8 oracle with unit scales must equal the
    bf16 oracle on the bf16 copy of the caches exactly, and with scales (powers of two keep the
    products exact) the bf16 oracle on pre-scaled copies."""
    from oracle import paged_decode_fp8_reference
    q, k8, v8, table, lens = _fp8_case(3, [1, 17, 40])
    kb, vb = k8.float().to(torch.bfloat16), v8.float().to(torch.bfloat16)
    assert torch.equal(kb.float(), k8.float()) and torch.equal(vb.float(), v8.float())
    a = paged_decode_fp8_reference(q, k8, v8, table, lens)
    b = paged_decode_reference(q, kb, vb, table, lens)
    assert torch.equal(a, b)
    a2 = paged_decode_fp8_reference(q, k8, v8, table, lens, k_scale=0.5, v_scale=4.0)
    b2 = paged_decode_reference(q, (kb.float() * 0.5).to(torch.bfloat16),
                                (vb.float() * 4.0).to(torch.bfloat16), table, lens)
    assert torch.allclose(a2, b2, atol=1e-5, rtol=1e-5)


def test_fp8_oracle_scales_are_not_swapped():
    """A planted mistake (k and v scales swapped) changes the result: k_scale sharpens the
    softmax, v_scale multiplies the output."""
    from oracle import paged_decode_fp8_reference
    q, k8, v8, table, lens = _fp8_case(4, [30, 50])
    a = paged_decode_fp8_reference(q, k8, v8, table, lens, k_scale=2.0, v_scale=0.5)
    swapped = paged_decode_fp8_reference(q, k8, v8, table, lens, k_scale=0.5, v_scale=2.0)
    assert not torch.allclose(a, swapped, atol=1e-3)
    unit = paged_decode_fp8_reference(q, k8, v8, table, lens, k_scale=2.0, v_scale=1.0)
    assert torch.allclose(a, unit * 0.5, atol=1e-6, rtol=1e-6)


def test_fp8_quantize_closed_form_codes():
    """fp8_quantize against codes the OCP e4m3fn format fixes by hand: 1 = 0x38, 448 = 0x7e
    (largest finite), saturation above it, 2^-9 = 0x01; ties go to the even code: 2^-10 -> 0,
    3 * 2^-10 -> 0x02, 1 + 1/16 -> 0x38 (1), 1 + 3/16 -> 0x3a (1.25); -0 keeps its sign; a
    scale divides first."""
    from oracle import fp8_quantize
    vals = [1.0, 448.0, 1000.0, -1000.0, 2.0 ** -9, 2.0 ** -10, 3 * 2.0 ** -10, 0.0, -0.0,
            1.0625, 1.1875, 464.0, -2.0 ** -9, 0.875]
    want = [0x38, 0x7E, 0x7E, 0xFE, 0x01, 0x00, 0x02, 0x00, 0x80, 0x38, 0x3A, 0x7E, 0x81, 0x36]
    x = torch.tensor(vals, dtype=torch.bfloat16)
    got = fp8_quantize(x, 1.0).view(torch.uint8).tolist()
    assert got == want, [hex(g) for g in got]
    assert fp8_quantize(torch.tensor([2.0, -896.0], dtype=torch.bfloat16), 2.0).view(
        torch.uint8).tolist() == [0x38, 0xFE]
    nan = fp8_quantize(torch.tensor([float("nan")], dtype=torch.bfloat16), 1.0).view(torch.uint8)
    assert int(nan[0]) & 0x7F == 0x7F
    inf = fp8_quantize(torch.tensor([float("inf"), -float("inf")], dtype=torch.bfloat16), 3.0)
    assert inf.view(torch.uint8).tolist() == [0x7E, 0xFE]


def test_fp8_quantize_round_trips_every_code_and_bounds_the_error():
    from oracle import fp8_dequantize, fp8_quantize
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    finite = [c for c in range(256) if (c & 0x7F) != 0x7F]
    vals = fp8_dequantize(codes.view(torch.float8_e4m3fn), 1.0)[finite]
    back = fp8_quantize(vals.to(torch.bfloat16), 1.0).view(torch.uint8)
    assert back.tolist() == finite
    # Rounding error of a normal value is at most half a step: |q - x| <= 2^-4 |x|.
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(4096, generator=g) * 20).to(torch.bfloat16)
    xf = x.float()
    q = fp8_dequantize(fp8_quantize(x, 1.0), 1.0)
    normal = xf.abs() >= 2.0 ** -6
    assert ((q - xf).abs()[normal] <= xf.abs()[normal] * 2.0 ** -4 + 1e-12).all()
    assert ((q - xf).abs()[~normal] <= 2.0 ** -10 + 1e-12).all()
