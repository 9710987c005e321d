"""Seeded synthetic inputs for the paged GQA decode operator.

Two families:
  * the five north-star configurations (tiny, Llama-3-8B decode, long context, ragged,
    large-shape sweep), with shuffled block tables;
  * the reference's 14-case contest table (task.md:110-127, confirmed copy
    bench_all.py:58-63) with its length recipe (bench_all.py:72-77: lengths uniform in
    [1, cap], sequence 0 at capacity, sequence 1 of length 1, case 1 all ones) and its
    consecutive block table (bench_all.py:81), optionally shuffled.

Generation order for one case is: seq_lens, block_table, q, k_cache, v_cache, all from one
``torch.Generator`` seeded with ``seed``.  q/K/V are N(0,1) drawn in fp32 (optionally scaled)
and rounded to bf16.  Small cases draw on the CPU generator, so their values do not depend on
the GPU; cases above ``CPU_GEN_LIMIT`` elements draw on the target device's generator.
"""

from __future__ import annotations

import math
import re
from dataclasses import dataclass, field, replace

import torch

CPU_GEN_LIMIT = 64 * 1024 * 1024   # K+V elements drawn on the CPU generator at most
_GEN_CHUNK = 32 * 1024 * 1024      # fp32 elements per generation chunk


@dataclass(frozen=True)
class DecodeSpec:
    """Shape and length recipe of one decode call."""

    name: str
    batch: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    page_size: int
    max_pages: int                 # block_table row width
    seq_lens: str = "fixed"        # fixed | uniform | loguniform_ragged | c500 | explicit
    seq_args: tuple = ()
    pool_pages: int = 0            # 0 -> batch * max_pages
    k_scale: float = 1.0
    table: str = "shuffle"         # shuffle | arange
    description: str = ""
    seqlen_q: int = 1              # query tokens per sequence (q is [B, Hq, D] when 1)
    causal: bool = False           # end-aligned causal mask for seqlen_q > 1

    @property
    def group(self) -> int:
        return self.num_heads // self.num_kv_heads

    @property
    def capacity(self) -> int:
        return self.max_pages * self.page_size

    @property
    def num_pages(self) -> int:
        return self.pool_pages or self.batch * self.max_pages

    def kv_elements(self) -> int:
        return 2 * self.num_pages * self.page_size * self.num_kv_heads * self.head_dim


@dataclass
class DecodeInputs:
    """Tensors of one decode call plus the spec that made them."""

    spec: DecodeSpec
    q: torch.Tensor            # [B, Hq, D] bf16
    k_cache: torch.Tensor      # [num_pages, P, Hkv, D] bf16
    v_cache: torch.Tensor
    block_table: torch.Tensor  # [B, max_pages] int32
    seq_lens: torch.Tensor     # [B] int32
    scale: float
    meta: dict = field(default_factory=dict)

    @property
    def device(self) -> torch.device:
        return self.q.device

    def kv_bytes(self) -> int:
        """Algorithmic K+V bytes of one call: sum_b L_b * Hkv * D * 2 (K, V) * 2 B."""
        return kv_bytes(self.seq_lens, self.spec.num_kv_heads, self.spec.head_dim)

    def to(self, device) -> "DecodeInputs":
        return replace(self, q=self.q.to(device), k_cache=self.k_cache.to(device),
                       v_cache=self.v_cache.to(device),
                       block_table=self.block_table.to(device),
                       seq_lens=self.seq_lens.to(device))

    def subset(self, batches) -> "DecodeInputs":
        """CPU copy holding only the given sequences and only their valid pages.

        Pages are gathered on the source device and renumbered 0..n-1, so a 16 GiB pool can
        be checked sequence by sequence on the host.
        """
        batches = [int(b) for b in batches]
        P = self.spec.page_size
        lens = self.seq_lens.cpu()[batches]
        table = self.block_table.cpu()[batches]
        npg = [max(1, math.ceil(int(L) / P)) for L in lens]
        ids = torch.cat([table[i, :n] for i, n in enumerate(npg)]).to(torch.long)
        k = self.k_cache.index_select(0, ids.to(self.k_cache.device)).cpu()
        v = self.v_cache.index_select(0, ids.to(self.v_cache.device)).cpu()
        width = max(npg)
        new_table = torch.zeros(len(batches), width, dtype=torch.int32)
        pos = 0
        for i, n in enumerate(npg):
            new_table[i, :n] = torch.arange(pos, pos + n, dtype=torch.int32)
            pos += n
        spec = replace(self.spec, batch=len(batches), max_pages=width, pool_pages=pos)
        return DecodeInputs(spec, self.q.cpu()[batches].contiguous(), k, v, new_table,
                            lens.clone(), self.scale, dict(self.meta, subset=batches))


def kv_bytes(seq_lens: torch.Tensor, num_kv_heads: int, head_dim: int) -> int:
    total = int(seq_lens.to(torch.int64).clamp(min=0).sum().item())
    return total * num_kv_heads * head_dim * 2 * 2


# ---------------------------------------------------------------------------------------
# North-star configurations
# ---------------------------------------------------------------------------------------

def _north_star_specs() -> dict[str, DecodeSpec]:
    s = {}
    s["tiny"] = DecodeSpec(
        "tiny", 4, 32, 8, 128, 16, 32, "uniform", (64, 512), pool_pages=256,
        description="config 1: B=4 Hq=32 Hkv=8 D=128 P=16, L~U[64,512], 256-page pool")
    s["llama3_8b"] = DecodeSpec(
        "llama3_8b", 64, 32, 8, 128, 16, 256, "fixed", (4096,),
        description="config 2: Llama-3-8B decode B=64 Hq=32 Hkv=8 D=128 P=16 L=4096")
    for B in (1, 4):
        for L in (32768, 131072):
            n = f"long_b{B}_{L // 1024}k"
            s[n] = DecodeSpec(
                n, B, 64, 8, 128, 16, L // 16, "fixed", (L,), k_scale=3.0,
                description=f"config 3: long context B={B} L={L} Hq=64 Hkv=8, K x3")
    s["ragged"] = DecodeSpec(
        "ragged", 256, 28, 4, 128, 64, 128, "loguniform_ragged", (1, 8192, 0.10, 15),
        description="config 4: ragged B=256 Hq=28 Hkv=4 (G=7) P=64, L log-uniform [1,8192], "
                    "10% in [1,15]")
    s["sweep_b32_16k"] = DecodeSpec(
        "sweep_b32_16k", 32, 64, 8, 128, 16, 1024, "fixed", (16384,),
        description="config 5: B=32 Hq=64 Hkv=8 D=128 L=16384")
    s["sweep_b128_16k"] = DecodeSpec(
        "sweep_b128_16k", 128, 64, 8, 128, 16, 1024, "fixed", (16384,),
        description="config 5: B=128 Hq=64 Hkv=8 D=128 L=16384")
    s["sweep_d64"] = DecodeSpec(
        "sweep_d64", 128, 32, 4, 64, 16, 512, "fixed", (8192,),
        description="config 5: D=64 Hq=32 Hkv=4 B=128 L=8192")
    s["sweep_d256"] = DecodeSpec(
        "sweep_d256", 64, 16, 2, 256, 16, 512, "fixed", (8192,),
        description="config 5: D=256 Hq=16 Hkv=2 B=64 L=8192")
    return s


NORTH_STAR = _north_star_specs()
BENCH_DEFAULT = "llama3_8b"   # the metric's quoted workload

# Measurement workloads beyond the north-star table: multi-token causal queries (speculative
# decode verification) on the Llama-3-8B decode shape.  4 draft tokens x group 4 fill one
# 16-row tile (same K/V traffic as the decode step); 8 tokens need two tiles.
EXTRA = {
    "specdec4_llama3_8b": DecodeSpec(
        "specdec4_llama3_8b", 64, 32, 8, 128, 16, 256, "fixed", (4096,), seqlen_q=4,
        causal=True, description="B=64 Hq=32 Hkv=8 D=128 P=16 L=4096, 4 causal query tokens"),
    "specdec8_llama3_8b": DecodeSpec(
        "specdec8_llama3_8b", 64, 32, 8, 128, 16, 256, "fixed", (4096,), seqlen_q=8,
        causal=True, description="B=64 Hq=32 Hkv=8 D=128 P=16 L=4096, 8 causal query tokens"),
    # Small query groups at config 2's bytes: one query head per KV head (MHA) and two.  The
    # MFMA tiles then hold 1 or 2 live rows of 16.
    "group1_llama3_8b": DecodeSpec(
        "group1_llama3_8b", 64, 8, 8, 128, 16, 256, "fixed", (4096,),
        description="B=64 Hq=8 Hkv=8 (group 1) D=128 P=16 L=4096"),
    "group2_llama3_8b": DecodeSpec(
        "group2_llama3_8b", 64, 16, 8, 128, 16, 256, "fixed", (4096,),
        description="B=64 Hq=16 Hkv=8 (group 2) D=128 P=16 L=4096"),
}

# The reference's case table: case -> (batch, seqlen_k capacity, num_heads_k)
# (bench_all.py:58-63; warmup/iters of bench_all.py:64).
C500_CASES = {
    1: (1, 1, 4), 2: (4, 2, 8), 3: (16, 17, 4), 4: (64, 64, 8), 5: (16, 141, 4),
    6: (16, 362, 8), 7: (64, 2048, 8), 8: (16, 4096, 4), 9: (32, 4096, 8), 10: (1, 8192, 4),
    11: (16, 12251, 4), 12: (8, 32768, 8), 13: (1, 58966, 8), 14: (1, 61519, 4),
}
C500_ITERS = {1: 100, 2: 100, 3: 100, 4: 50, 5: 50, 6: 50, 7: 12, 8: 25, 9: 12, 10: 25,
              11: 12, 12: 12, 13: 25, 14: 25}


def c500_spec(case: int, table: str = "arange") -> DecodeSpec:
    batch, cap, kv = C500_CASES[case]
    pages = math.ceil(cap / 16)
    return DecodeSpec(f"c500_case{case}", batch, 32, kv, 128, 16, pages, "c500", (cap, case),
                      table=table, description=f"contest case {case}: b{batch} cap{cap} kv{kv}")


_SHAPE_NAME = re.compile(r"(uniform|ragged)_b(\d+)_hq(\d+)_hkv(\d+)_l(\d+)(?:_d(\d+))?")


def shape_spec(kind: str, batch: int, num_heads: int, num_kv_heads: int, length: int,
               head_dim: int = 128) -> DecodeSpec:
    """Page_size 16 decode of `batch` sequences (head_dim 128 unless a `_d<D>` suffix says
    otherwise): every one `length` keys ("uniform"), or config 4's recipe up to `length`
    ("ragged": log-uniform in [1, length], 10 % in [1, 15])."""
    pages = math.ceil(length / 16)
    name = f"{kind}_b{batch}_hq{num_heads}_hkv{num_kv_heads}_l{length}"
    if head_dim != 128:
        name += f"_d{head_dim}"
    if kind == "uniform":
        return DecodeSpec(name, batch, num_heads, num_kv_heads, head_dim, 16, pages, "fixed",
                          (length,), description=f"uniform B={batch} Hq={num_heads} "
                                                 f"Hkv={num_kv_heads} L={length} D={head_dim}")
    if kind == "ragged":
        return DecodeSpec(name, batch, num_heads, num_kv_heads, head_dim, 16, pages,
                          "loguniform_ragged", (1, length, 0.10, 15),
                          description=f"ragged B={batch} Hq={num_heads} Hkv={num_kv_heads} "
                                      f"L log-uniform [1,{length}], 10% in [1,15]")
    raise ValueError(f"unknown shape kind {kind!r}")


def get_spec(name: str) -> DecodeSpec:
    if name in NORTH_STAR:
        return NORTH_STAR[name]
    if name in EXTRA:
        return EXTRA[name]
    if name.startswith("c500_case"):
        return c500_spec(int(name[len("c500_case"):]))
    m = _SHAPE_NAME.fullmatch(name)
    if m:
        return shape_spec(m.group(1), *(int(x) for x in m.groups()[1:5]),
                          head_dim=int(m.group(6)) if m.group(6) else 128)
    raise KeyError(f"unknown workload {name!r}; known: {sorted(NORTH_STAR)}, c500_case1..14, "
                   "uniform_bB_hqH_hkvK_lL and ragged_bB_hqH_hkvK_lL (optional _dD suffix)")


# ---------------------------------------------------------------------------------------
# Generation
# ---------------------------------------------------------------------------------------

def _make_seq_lens(spec: DecodeSpec, gen: torch.Generator) -> torch.Tensor:
    B = spec.batch
    kind, a = spec.seq_lens, spec.seq_args
    if kind == "fixed":
        lens = torch.full((B,), int(a[0]), dtype=torch.int32)
    elif kind == "uniform":
        lens = torch.randint(int(a[0]), int(a[1]) + 1, (B,), generator=gen, dtype=torch.int32)
    elif kind == "loguniform_ragged":
        lo, hi, frac, short_hi = a
        u = torch.rand(B, generator=gen, dtype=torch.float64)
        lens = torch.exp(math.log(lo) + u * (math.log(hi + 1) - math.log(lo))).floor()
        lens = lens.clamp(lo, hi).to(torch.int32)
        n_short = max(1, int(round(frac * B)))
        idx = torch.randperm(B, generator=gen)[:n_short]
        lens[idx] = torch.randint(1, int(short_hi) + 1, (n_short,), generator=gen,
                                  dtype=torch.int32)
    elif kind == "c500":
        cap, case = a
        if case == 1:
            lens = torch.ones(B, dtype=torch.int32)
        else:
            lens = torch.randint(1, cap + 1, (B,), generator=gen, dtype=torch.int32)
            lens[0] = cap
            if B > 1:
                lens[1] = 1
    elif kind == "explicit":
        lens = torch.tensor([int(x) for x in a], dtype=torch.int32)
    else:
        raise ValueError(f"unknown seq_lens recipe {kind!r}")
    return lens


def _make_table(spec: DecodeSpec, gen: torch.Generator) -> torch.Tensor:
    need = spec.batch * spec.max_pages
    if spec.num_pages < need:
        raise ValueError(f"pool of {spec.num_pages} pages is smaller than B*max_pages={need}")
    if spec.table == "arange":
        ids = torch.arange(need, dtype=torch.int32)
    else:
        ids = torch.randperm(spec.num_pages, generator=gen)[:need].to(torch.int32)
    return ids.view(spec.batch, spec.max_pages).contiguous()


def _randn_bf16(shape, gen: torch.Generator, gen_device, out_device, scale: float = 1.0):
    out = torch.empty(shape, dtype=torch.bfloat16, device=out_device)
    flat = out.view(-1)
    n = flat.numel()
    for s in range(0, n, _GEN_CHUNK):
        m = min(_GEN_CHUNK, n - s)
        t = torch.randn(m, generator=gen, device=gen_device, dtype=torch.float32)
        if scale != 1.0:
            t.mul_(scale)
        flat[s:s + m].copy_(t.to(torch.bfloat16))
    return out


def make_inputs(spec: DecodeSpec | str, seed: int = 0, device="cpu",
                gen_device=None) -> DecodeInputs:
    """Build the tensors of one decode call on ``device``."""
    if isinstance(spec, str):
        spec = get_spec(spec)
    device = torch.device(device)
    if gen_device is None:
        gen_device = "cpu" if spec.kv_elements() <= CPU_GEN_LIMIT else device
    gen_device = torch.device(gen_device)
    cpu_gen = torch.Generator(device="cpu").manual_seed(seed)
    lens = _make_seq_lens(spec, cpu_gen)
    table = _make_table(spec, cpu_gen)
    if gen_device.type == "cpu":
        gen = cpu_gen
    else:
        gen = torch.Generator(device=gen_device).manual_seed(seed)
    q_shape = ((spec.batch, spec.num_heads, spec.head_dim) if spec.seqlen_q == 1 else
               (spec.batch, spec.seqlen_q, spec.num_heads, spec.head_dim))
    q = _randn_bf16(q_shape, gen, gen_device, device)
    kv_shape = (spec.num_pages, spec.page_size, spec.num_kv_heads, spec.head_dim)
    k = _randn_bf16(kv_shape, gen, gen_device, device, spec.k_scale)
    v = _randn_bf16(kv_shape, gen, gen_device, device)
    return DecodeInputs(spec, q, k, v, table.to(device), lens.to(device),
                        1.0 / math.sqrt(spec.head_dim),
                        {"seed": seed, "gen_device": str(gen_device)})


def custom_spec(name: str, seq_lens, num_heads: int, num_kv_heads: int, head_dim: int,
                page_size: int, max_pages: int | None = None, pool_pages: int = 0,
                table: str = "shuffle", k_scale: float = 1.0, seqlen_q: int = 1,
                causal: bool = False) -> DecodeSpec:
    """Spec with explicit per-sequence lengths (edge-case tests)."""
    lens = [int(x) for x in seq_lens]
    if max_pages is None:
        max_pages = max(1, max(math.ceil(max(L, 1) / page_size) for L in lens))
    return DecodeSpec(name, len(lens), num_heads, num_kv_heads, head_dim, page_size, max_pages,
                      "explicit", tuple(lens), pool_pages=pool_pages, table=table,
                      k_scale=k_scale, seqlen_q=seqlen_q, causal=causal)
