"""Synthetic workload recipes: shapes of the north-star configurations and of the reference's
14-case table (task.md:110-127, bench_all.py:58-81), determinism, and the subset helper the
large-configuration parity tests rely on."""

from __future__ import annotations

import math

import pytest
import torch

from mx_flash_attn_kernel_opt__amd import workloads as W
from oracle import kv_bytes, paged_decode_reference


def test_north_star_shapes():
    s = W.NORTH_STAR
    assert (s["tiny"].batch, s["tiny"].num_heads, s["tiny"].num_kv_heads, s["tiny"].head_dim,
            s["tiny"].page_size, s["tiny"].num_pages) == (4, 32, 8, 128, 16, 256)
    l8 = s["llama3_8b"]
    assert (l8.batch, l8.num_heads, l8.num_kv_heads, l8.head_dim, l8.page_size) == \
        (64, 32, 8, 128, 16)
    assert l8.num_pages == 64 * 256 and l8.seq_args == (4096,)
    for B in (1, 4):
        for L in (32768, 131072):
            c = s[f"long_b{B}_{L // 1024}k"]
            assert (c.batch, c.num_heads, c.num_kv_heads, c.capacity, c.k_scale) == \
                (B, 64, 8, L, 3.0)
    r = s["ragged"]
    assert (r.batch, r.num_heads, r.num_kv_heads, r.page_size, r.capacity) == \
        (256, 28, 4, 64, 8192)
    assert (s["sweep_d64"].head_dim, s["sweep_d64"].num_heads, s["sweep_d64"].num_kv_heads,
            s["sweep_d64"].batch) == (64, 32, 4, 128)
    assert (s["sweep_d256"].head_dim, s["sweep_d256"].num_heads, s["sweep_d256"].num_kv_heads,
            s["sweep_d256"].batch) == (256, 16, 2, 64)
    assert s["sweep_b128_16k"].capacity == 16384 and s["sweep_b32_16k"].batch == 32


def test_llama_kv_bytes_is_one_gib():
    spec = W.NORTH_STAR["llama3_8b"]
    lens = torch.full((spec.batch,), 4096, dtype=torch.int32)
    assert kv_bytes(lens, spec.num_kv_heads, spec.head_dim) == 1 << 30
    assert W.kv_bytes(lens, spec.num_kv_heads, spec.head_dim) == 1 << 30


def test_generation_is_deterministic_and_seeded():
    a = W.make_inputs("tiny", seed=0)
    b = W.make_inputs("tiny", seed=0)
    c = W.make_inputs("tiny", seed=1)
    for x, y in ((a.q, b.q), (a.k_cache, b.k_cache), (a.block_table, b.block_table),
                 (a.seq_lens, b.seq_lens)):
        assert torch.equal(x, y)
    assert not torch.equal(a.k_cache, c.k_cache)
    assert a.q.dtype == torch.bfloat16 and a.block_table.dtype == torch.int32
    lens = a.seq_lens
    assert ((lens >= 64) & (lens <= 512)).all()
    ids = a.block_table.flatten()
    assert len(set(ids.tolist())) == ids.numel() and int(ids.max()) < 256


def test_ragged_recipe():
    spec = W.NORTH_STAR["ragged"]
    gen = torch.Generator().manual_seed(0)
    lens = W._make_seq_lens(spec, gen)
    assert lens.shape == (256,) and int(lens.min()) >= 1 and int(lens.max()) <= 8192
    assert int((lens <= 15).sum()) >= 25       # 10% forced to 1..15 tokens
    assert int((lens > 1024).sum()) > 20       # the log-uniform bulk reaches long lengths
    table = W._make_table(spec, gen)
    assert table.shape == (256, 128)
    assert len(set(table.flatten().tolist())) == 256 * 128


def test_named_shapes():
    u = W.get_spec("uniform_b16_hq32_hkv8_l4096")
    assert (u.batch, u.num_heads, u.num_kv_heads, u.head_dim, u.page_size) == (16, 32, 8, 128, 16)
    assert u.capacity == 4096
    lens = W.make_inputs(u, seed=3).seq_lens
    assert lens.tolist() == [4096] * 16
    r = W.get_spec("ragged_b8_hq64_hkv8_l8192")
    assert (r.batch, r.num_heads, r.num_kv_heads, r.capacity) == (8, 64, 8, 8192)
    lens = W.make_inputs(r, seed=3).seq_lens
    assert int(lens.min()) >= 1 and int(lens.max()) <= 8192 and len(set(lens.tolist())) > 1
    with pytest.raises(KeyError):
        W.get_spec("uniform_b16_hq32_l4096")


@pytest.mark.parametrize("case", range(1, 15))
def test_c500_case_recipe(case):
    spec = W.c500_spec(case)
    B, cap, kv = W.C500_CASES[case]
    assert (spec.batch, spec.num_kv_heads, spec.num_heads, spec.head_dim, spec.page_size) == \
        (B, kv, 32, 128, 16)
    assert spec.max_pages == math.ceil(cap / 16)
    lens = W._make_seq_lens(spec, torch.Generator().manual_seed(42))
    if case == 1:
        assert lens.tolist() == [1] * B
    else:
        assert int(lens[0]) == cap and int(lens.max()) <= cap and int(lens.min()) >= 1
        if B > 1:
            assert int(lens[1]) == 1
    table = W._make_table(spec, torch.Generator())
    assert torch.equal(table.flatten(), torch.arange(B * spec.max_pages, dtype=torch.int32))


def test_subset_keeps_the_oracle_result():
    inp = W.make_inputs("tiny", seed=3)
    full = paged_decode_reference(inp.q, inp.k_cache, inp.v_cache, inp.block_table,
                                  inp.seq_lens, inp.scale)
    sub = inp.subset([2, 0])
    assert sub.k_cache.shape[0] == sum(math.ceil(int(L) / 16) for L in inp.seq_lens[[2, 0]])
    part = paged_decode_reference(sub.q, sub.k_cache, sub.v_cache, sub.block_table,
                                  sub.seq_lens, sub.scale)
    assert torch.equal(part, full[[2, 0]])
