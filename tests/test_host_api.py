"""Host-side checks of libmxattn.so that need no GPU.

* the library loads and exports every function include/mx_paged_decode.h declares;
* argument validation returns the documented status before any HIP call (reference
  run_kernel validates nothing, submission_clean.cu:432-504; the original LSE kernel silently
  returns on unsupported shapes, optimized_c500_flash_attn.cu:890-900);
* the split planner (replacing submission_clean.cu:375-430, 456-461) keeps its invariants.
"""

from __future__ import annotations

import ctypes
import math
import os
import re
import subprocess

import pytest

from conftest import gpu_available
from mx_flash_attn_kernel_opt__amd import MXAttnError, _lib, plan
from mx_flash_attn_kernel_opt__amd import workloads as W

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "mx_paged_decode.h")


def header_functions() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?(?:void|int|int64_t|char)\s*\*?\s*(\w+)\s*\(",
                      text, flags=re.M)


def test_header_declares_the_drop_in_and_extended_entry_points():
    fns = header_functions()
    for name in ("run_kernel", "mx_paged_gqa_decode", "mx_paged_gqa_decode_plan",
                 "mx_paged_gqa_decode_workspace_size", "mx_read_device_status",
                 "mx_last_status", "mx_last_error", "mx_version"):
        assert name in fns
    assert set(fns) == set(_lib.SIGNATURES), "ctypes binding and header disagree"


def test_library_exports_every_header_symbol():
    lib = _lib.load()
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.library_path()],
                         capture_output=True, text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if ln.strip()}
    for name in header_functions():
        assert name in exported, f"{name} not exported"
        assert getattr(lib, name) is not None
    assert b"gfx950" in lib.mx_version()


def test_run_kernel_abi_matches_the_reference_binding():
    # verify_real.py:12-14: argtypes [c_void_p]*6 + [c_int64]*9, restype None
    restype, argtypes = _lib.SIGNATURES["run_kernel"]
    assert restype is None
    assert argtypes == [ctypes.c_void_p] * 6 + [ctypes.c_int64] * 9


# ------------------------------------------------------------------------------------------
# Validation (no HIP call is reached on these paths)
# ------------------------------------------------------------------------------------------

FAKE = ctypes.c_void_p(0x1000)   # never dereferenced: validation fails first
PARTIAL_BASE = 256 + 128 * 256 + 4 * (4096 + 8192) * 4   # status word, XCD claim masks, merge counters


def _decode(**over):
    args = dict(q=FAKE, k=FAKE, v=FAKE, out=FAKE, lens=FAKE, table=FAKE, B=2, SQ=1, Hq=32,
                Hkv=8, D=128, P=16, pages=64, max_pages=32, max_seq=0, causal=0, scale=0.088,
                ns=2, ws=FAKE, ws_bytes=1 << 30, phase=0, stream=None)
    args.update(over)
    lib = _lib.load()
    return lib.mx_paged_gqa_decode(args["q"], args["k"], args["v"], args["out"], args["lens"],
                                   args["table"], args["B"], args["SQ"], args["Hq"], args["Hkv"],
                                   args["D"], args["P"], args["pages"], args["max_pages"],
                                   args["max_seq"], args["causal"], args["scale"], args["ns"],
                                   args["ws"], args["ws_bytes"], args["phase"], args["stream"])


@pytest.mark.parametrize("field", ["q", "k", "v", "out", "lens", "table"])
def test_null_pointers_are_rejected(field):
    assert _decode(**{field: None}) == _lib.MX_STATUS_NULL_POINTER
    assert "non-NULL" in _lib.load().mx_last_error().decode()


@pytest.mark.parametrize("over,status", [
    (dict(Hq=30, Hkv=8), _lib.MX_STATUS_INVALID_SHAPE),
    (dict(B=0), _lib.MX_STATUS_INVALID_SHAPE),
    (dict(Hkv=0), _lib.MX_STATUS_INVALID_SHAPE),
    (dict(max_pages=0), _lib.MX_STATUS_INVALID_SHAPE),
    (dict(pages=-1), _lib.MX_STATUS_INVALID_SHAPE),
    (dict(ns=-3, B=600), _lib.MX_STATUS_UNSUPPORTED),     # balanced schedule: batch <= 512
    (dict(ns=-3, B=500, Hq=32, Hkv=32), _lib.MX_STATUS_UNSUPPORTED),   # batch * Hkv <= 8192
    (dict(D=96), _lib.MX_STATUS_UNSUPPORTED),
    (dict(D=512), _lib.MX_STATUS_UNSUPPORTED),
    (dict(P=8), _lib.MX_STATUS_UNSUPPORTED),
    (dict(P=48), _lib.MX_STATUS_UNSUPPORTED),
    (dict(Hq=512, Hkv=2), _lib.MX_STATUS_UNSUPPORTED),    # group 256 > 128
    (dict(B=70000), _lib.MX_STATUS_UNSUPPORTED),
    (dict(SQ=0), _lib.MX_STATUS_INVALID_SHAPE),
    (dict(B=300, SQ=300), _lib.MX_STATUS_UNSUPPORTED),    # combine grid: batch * seqlen_q
    (dict(causal=2), _lib.MX_STATUS_INVALID_ARGUMENT),
    (dict(ns=-3, B=512, Hkv=8, Hq=128, SQ=8), _lib.MX_STATUS_UNSUPPORTED),  # 16384 units
    (dict(phase=3), _lib.MX_STATUS_INVALID_ARGUMENT),
    (dict(scale=float("nan")), _lib.MX_STATUS_INVALID_ARGUMENT),
    (dict(scale=float("inf")), _lib.MX_STATUS_INVALID_ARGUMENT),
    (dict(ws_bytes=100), _lib.MX_STATUS_WORKSPACE_TOO_SMALL),
    (dict(q=ctypes.c_void_p(0x1008)), _lib.MX_STATUS_INVALID_ARGUMENT),   # 16-byte loads
    (dict(k=ctypes.c_void_p(0x1004)), _lib.MX_STATUS_INVALID_ARGUMENT),
    (dict(v=ctypes.c_void_p(0x1002)), _lib.MX_STATUS_INVALID_ARGUMENT),
    (dict(out=ctypes.c_void_p(0x1004)), _lib.MX_STATUS_INVALID_ARGUMENT),  # 8-byte stores
])
def test_invalid_arguments_return_status(over, status):
    assert _decode(**over) == status
    assert _lib.load().mx_last_status() == status
    assert _lib.load().mx_last_error()


def _run_kernel(**over):
    a = dict(B=4, seqlen_k=512, seqlen_q=1, Hq=32, Hkv=8, D=128, P=16, nb=128, causal=0)
    a.update(over)
    lib = _lib.load()
    lib.run_kernel(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, a["B"], a["seqlen_k"], a["seqlen_q"],
                   a["Hq"], a["Hkv"], a["D"], a["P"], a["nb"], a["causal"])
    return lib.mx_last_status()


@pytest.mark.parametrize("over,status", [
    (dict(seqlen_q=0), _lib.MX_STATUS_INVALID_SHAPE),
    (dict(causal=2), _lib.MX_STATUS_INVALID_ARGUMENT),
    (dict(nb=130), _lib.MX_STATUS_INVALID_SHAPE),
    (dict(nb=2), _lib.MX_STATUS_INVALID_SHAPE),
    (dict(seqlen_k=0), _lib.MX_STATUS_INVALID_SHAPE),
    (dict(Hq=32, Hkv=5), _lib.MX_STATUS_INVALID_SHAPE),
    (dict(D=100), _lib.MX_STATUS_UNSUPPORTED),
])
def test_run_kernel_rejects_what_the_reference_ignores(over, status, capfd):
    assert _run_kernel(**over) == status
    assert "run_kernel" in capfd.readouterr().err


@pytest.mark.skipif(gpu_available(), reason="checks the no-device path")
def test_automatic_plan_without_a_device_reports_hip_error():
    assert _decode(ns=0) == _lib.MX_STATUS_HIP_ERROR


def test_python_wrapper_raises_with_status():
    with pytest.raises(MXAttnError) as e:
        plan(2, 30, 8, 128, 16, 32, num_cus=256)
    assert e.value.status == _lib.MX_STATUS_INVALID_SHAPE


# ------------------------------------------------------------------------------------------
# Planner invariants
# ------------------------------------------------------------------------------------------

@pytest.mark.parametrize("B,Hq,Hkv,D,P,max_pages,cap,ns_req", [
    (64, 32, 8, 128, 16, 256, 0, 3),
    (1, 64, 8, 128, 16, 8192, 0, 64),
    (256, 28, 4, 128, 64, 128, 0, 5),
    (4, 32, 8, 128, 16, 32, 512, 2),
    (3, 32, 8, 128, 16, 40, 300, 7),
    (8, 32, 8, 64, 32, 100, 0, 7),
    (2, 16, 2, 256, 16, 10, 0, 1000),
    (1, 32, 4, 128, 16, 1, 1, 1),
    (600, 32, 8, 128, 16, 64, 0, 0),      # automatic plan above the balanced batch limit
])
def test_split_grid_plan_invariants(B, Hq, Hkv, D, P, max_pages, cap, ns_req):
    p = plan(B, Hq, Hkv, D, P, max_pages, cap, ns_req, num_cus=256)
    assert p["schedule"] == "split_grid"
    ns, tps, ws = p["splits"], p["tokens_per_split"], p["workspace_bytes"]
    table_tokens = max_pages * P
    eff_cap = cap if 0 < cap < table_tokens else table_tokens
    cap_pages = math.ceil(eff_cap / P)
    assert 1 <= ns <= cap_pages
    assert tps % P == 0 and tps >= P
    assert ns * tps >= eff_cap                      # every capacity token is covered
    assert (ns - 1) * tps < eff_cap                 # and no split is empty at capacity
    assert p["workgroups"] == B * Hkv * ns
    if ns_req > 0:
        assert ns <= ns_req
    if ns == 1:
        assert ws == 256
    else:
        rows = B * Hq * ns
        assert ws == PARTIAL_BASE + math.ceil(rows * 4 / 256) * 256 + rows * D * 4


@pytest.mark.parametrize("B,Hq,Hkv,D,ns_req,groups,paired", [
    (64, 32, 8, 128, 0, 256, True),      # automatic: one 4-wave workgroup per CU at D=128
    (128, 32, 4, 64, 0, 512, False),     # two 2-wave workgroups per CU at D=64
    (64, 16, 2, 256, 0, 256, False),     # one per CU at D=256
    (4, 32, 8, 128, -7, 7, False),       # forced workgroup count: never paired
    (512, 28, 4, 128, 0, 256, True),     # 4 KV heads: mirrored pairs, more pairs than groups
    (128, 28, 4, 128, 0, 256, False),    # 4 KV heads, as many pairs as groups: single heads
    (192, 28, 2, 128, 0, 256, False),    # 2 KV heads (512-byte token rows): single heads
    (3, 32, 8, 128, -9000, 4095, False),  # clamped to the 8^4 merge tree
    (32, 128, 16, 128, 0, 256, True),    # 16 KV heads, group 8: pairs of 16 rows
])
def test_balanced_plan(B, Hq, Hkv, D, ns_req, groups, paired):
    """Slots of the balanced schedule: one per workgroup and one per unit, of min(rows, 16)
    rows; paired units are two KV heads (adjacent, or heads 0 and 3, 1 and 2 of four) with both
    heads' rows."""
    p = plan(B, Hq, Hkv, D, 16, 256, 0, ns_req, num_cus=256)
    assert p["schedule"] == ("balanced_paired" if paired else "balanced")
    assert p["workgroups"] == groups and p["splits"] == 0
    slots = groups + B * Hkv // (2 if paired else 1)
    G = Hq // Hkv * (2 if paired else 1)
    o_off = PARTIAL_BASE + math.ceil(slots * G * 4 / 256) * 256
    assert p["workspace_bytes"] == o_off + slots * G * D * 4


def test_policy_on_the_north_star_configs():
    """The automatic plan on a 256-CU MI355X (from interleaved A/B sweeps): batches of at
    least 64 (sequence, KV head) units take the balanced single launch; fewer, long units take
    the split grid with about one workgroup per CU, over pairs of KV heads where each paired
    split keeps at least 896 tokens."""
    expect = {
        "tiny": ("split_grid", 4), "llama3_8b": ("balanced_paired", 256),
        "long_b1_32k": ("split_grid", 32), "long_b1_128k": ("split_grid_paired", 64),
        "long_b4_32k": ("split_grid_paired", 16), "long_b4_128k": ("split_grid_paired", 16),
        "ragged": ("balanced_paired", 256), "sweep_b32_16k": ("balanced_paired", 256),
        "sweep_b128_16k": ("balanced_paired", 256), "sweep_d64": ("balanced", 512),
        "sweep_d256": ("balanced", 256),
    }
    for name, s in W.NORTH_STAR.items():
        p = plan(s.batch, s.num_heads, s.num_kv_heads, s.head_dim, s.page_size, s.max_pages,
                 num_cus=256)
        sched, n = expect[name]
        assert p["schedule"] == sched, name
        assert (p["workgroups"] if sched.startswith("balanced") else p["splits"]) == n, name


@pytest.mark.parametrize("B,Hq,Hkv,D,cap,sq,fp8,ns_req,sched,splits", [
    (1, 64, 8, 128, 131072, 1, False, 0, "split_grid_paired", 64),
    (4, 64, 8, 128, 32768, 1, False, 0, "split_grid_paired", 16),
    (1, 64, 8, 128, 32768, 1, False, 0, "split_grid", 32),    # paired splits of 512 tokens
    (1, 32, 8, 128, 58976, 1, False, 0, "split_grid_paired", 64),  # 928 tokens (case 13)
    (1, 64, 8, 128, 131072, 1, True, 0, "split_grid_paired", 64),  # fp8: 1 KB token rows
    (1, 64, 8, 128, 131072, 1, False, 32, "split_grid", 32),  # explicit split counts are not
    (1, 56, 7, 128, 131072, 1, False, 0, "split_grid", 37),   # odd KV head count
    (1, 64, 4, 128, 131072, 1, False, 0, "split_grid", 64),   # group 16: 32 rows per pair
    (1, 32, 8, 128, 131072, 2, False, 0, "split_grid_paired", 64),  # 2 tokens x group 4
    (1, 32, 8, 128, 131072, 3, False, 0, "split_grid", 32),   # 3 x 4 x 2 = 24 rows
    (1, 32, 8, 64, 131072, 1, False, 0, "split_grid", 64),    # head_dim 64
    (1, 16, 4, 256, 131072, 1, False, 0, "split_grid", 64),   # head_dim 256
])
def test_paired_split_grid_plan(B, Hq, Hkv, D, cap, sq, fp8, ns_req, sched, splits):
    """Pairs of adjacent KV heads share a workgroup on the automatic split grid (bf16 cache,
    head_dim 128, an even KV head count, 2 * seqlen_q * group <= 16, paired splits of at least
    896 tokens): units of two heads, about one workgroup per CU, the same partial rows."""
    p = plan(B, Hq, Hkv, D, 16, cap // 16, 0, ns_req, num_cus=256, seqlen_q=sq, fp8=fp8)
    assert p["schedule"] == sched and p["splits"] == splits
    units = B * (Hkv // 2 if sched == "split_grid_paired" else Hkv)
    row_groups = 1 if sched == "split_grid_paired" else math.ceil(sq * Hq // Hkv / 16 / (
        2 if sq * Hq // Hkv > 16 and D <= 128 else 1))
    assert p["workgroups"] == units * row_groups * splits
    prow = B * sq * Hq * splits
    assert p["workspace_bytes"] == PARTIAL_BASE + math.ceil(prow * 4 / 256) * 256 + prow * D * 4
    assert p["launches"] == 1
    if sched == "split_grid_paired":
        assert p["tokens_per_split"] >= 896


@pytest.mark.parametrize("B,Hq,Hkv,cap,sq,fp8,sched,units", [
    (48, 20, 10, 8192, 1, False, "balanced_paired", 240),   # 5 pairs per sequence
    (48, 40, 10, 8192, 2, False, "balanced_paired", 240),   # 2 tokens x group 4 x 2 heads
    (2, 20, 10, 32768, 1, False, "split_grid_paired", 10),
    (2, 40, 10, 32768, 2, False, "split_grid_paired", 10),
    (48, 24, 12, 8192, 1, False, "balanced_paired", 288),   # 6 pairs
    (2, 24, 12, 32768, 1, False, "split_grid_paired", 12),
    (96, 12, 6, 4096, 1, True, "balanced_paired", 288),     # fp8, 3 pairs of 512-byte rows
    (128, 24, 6, 4096, 2, True, "balanced_paired", 384),
    (96, 12, 6, 4096, 1, False, "balanced", 576),           # bf16 1.5 KB rows: not paired
    (40, 24, 6, 4096, 1, True, "balanced", 240),            # fp8: fewer pair units than groups
])
def test_odd_pair_counts_plan(B, Hq, Hkv, cap, sq, fp8, sched, units):
    """Automatic plans over an odd number of KV-head pairs per sequence (5 or 3) and an even
    one (6): paired units are B * Hkv / 2, with both heads' rows in one slot; the balanced
    plan's slots are one per workgroup and one per unit."""
    p = plan(B, Hq, Hkv, 128, 16, cap // 16, cap, 0, num_cus=256, seqlen_q=sq, fp8=fp8)
    assert p["schedule"] == sched
    paired = sched.endswith("_paired")
    assert units == B * (Hkv // 2 if paired else Hkv)
    if sched.startswith("balanced"):
        assert p["workgroups"] == 256
        rows = sq * Hq // Hkv * (2 if paired else 1)
        slots = 256 + units
        o_off = PARTIAL_BASE + math.ceil(slots * rows * 4 / 256) * 256
        assert p["workspace_bytes"] == o_off + slots * rows * 128 * 4
    else:
        assert p["workgroups"] == units * p["splits"] and p["tokens_per_split"] >= 1024
        assert p["launches"] == 1


@pytest.mark.parametrize("B,Hkv,cap,sched,splits", [
    (64, 8, 64, "split_grid", 1),       # short capacity: one split per unit, no merge
    (64, 8, 512, "split_grid", 1),
    (16, 4, 141, "split_grid", 1),      # 141 tokens: a second split would hold < 128
    (16, 4, 512, "split_grid", 4),      # 64 units: four 128-token splits fill the CUs
    (64, 4, 1024, "split_grid", 1),     # 1 024 tokens with 256 units: split grid
    (64, 8, 1024, "balanced_paired", 0),  # ... with 512 units: balanced (8 heads: paired)
    (16, 8, 2048, "balanced_paired", 0),  # from 2 048 tokens: balanced
])
def test_policy_capacity_gate(B, Hkv, cap, sched, splits):
    """Batches of short sequences skip the balanced schedule (its length scan and merges cost
    more than the imbalance they remove below ~2 048 tokens of capacity)."""
    p = plan(B, 32, Hkv, 128, 16, 512, cap, 0, num_cus=256)
    assert p["schedule"] == sched
    assert p["splits"] == splits


@pytest.mark.parametrize("SQ,Hq,Hkv,D,groups,group_rows", [
    (1, 32, 8, 128, 1, 4), (4, 32, 8, 128, 1, 16), (5, 32, 8, 128, 1, 20), (8, 64, 8, 128, 2, 32),
    (16, 8, 8, 128, 1, 16), (17, 8, 8, 128, 1, 17), (3, 28, 4, 64, 1, 21),
    (5, 32, 8, 256, 2, 16),    # head_dim 256: single 16-row tiles only
])
def test_multi_token_row_groups(SQ, Hq, Hkv, D, groups, group_rows):
    """seqlen_q * group query rows per KV head run in row groups: one 16-row tile, or (above
    16 rows, head_dim <= 128) two tiles sharing each pass over K/V.  The split grid launches
    Hkv * groups workgroups per (sequence, split), its partial rows are per (token, head), and
    the balanced schedule counts one unit per (sequence, KV head, row group) with partial
    slots of min(rows, rows per group) rows."""
    p = plan(2, Hq, Hkv, D, 16, 64, 0, 3, num_cus=256, seqlen_q=SQ)
    assert p["schedule"] == "split_grid" and p["splits"] == 3
    assert p["workgroups"] == 2 * Hkv * groups * 3
    rows = 2 * SQ * Hq * 3
    assert p["workspace_bytes"] == PARTIAL_BASE + math.ceil(rows * 4 / 256) * 256 + rows * D * 4
    b = plan(64, Hq, Hkv, D, 16, 64, 0, -100, num_cus=256, seqlen_q=SQ)
    slots = 100 + 64 * Hkv * groups
    assert b["schedule"] == "balanced"
    assert b["workspace_bytes"] == (PARTIAL_BASE + math.ceil(slots * group_rows * 4 / 256) * 256
                                    + slots * group_rows * D * 4)


@pytest.mark.skipif(gpu_available(), reason="would launch on the fake pointers")
def test_run_kernel_accepts_multi_token_causal_arguments():
    """seqlen_q > 1 and causal = 1 pass validation: without a device the call gets as far as
    the device query."""
    assert _run_kernel(seqlen_q=4, causal=1) == _lib.MX_STATUS_HIP_ERROR


# ------------------------------------------------------------------------------------------
# Paged K/V append: validation (no HIP call is reached on these paths)
# ------------------------------------------------------------------------------------------

def _append(**over):
    a = dict(kn=FAKE, vn=FAKE, k=FAKE, v=FAKE, lens=FAKE, table=FAKE, B=4, S=1, Hkv=8, D=128,
             P=16, pages=64, max_pages=16, ws=None, stream=None)
    a.update(over)
    return _lib.load().mx_paged_kv_append(a["kn"], a["vn"], a["k"], a["v"], a["lens"],
                                          a["table"], a["B"], a["S"], a["Hkv"], a["D"], a["P"],
                                          a["pages"], a["max_pages"], a["ws"], a["stream"])


@pytest.mark.parametrize("over,status", [
    (dict(kn=None), _lib.MX_STATUS_NULL_POINTER),
    (dict(table=None), _lib.MX_STATUS_NULL_POINTER),
    (dict(v=ctypes.c_void_p(0x1008)), _lib.MX_STATUS_INVALID_ARGUMENT),   # not 16-byte aligned
    (dict(pages=0), _lib.MX_STATUS_INVALID_SHAPE),                        # pool size required
    (dict(B=0), _lib.MX_STATUS_INVALID_SHAPE),
    (dict(S=-1), _lib.MX_STATUS_INVALID_SHAPE),
    (dict(D=100), _lib.MX_STATUS_UNSUPPORTED),
    (dict(max_pages=1 << 28, P=16), _lib.MX_STATUS_UNSUPPORTED),
])
def test_append_rejects_invalid_arguments(over, status):
    assert _append(**over) == status
    assert _lib.load().mx_last_error()


def test_append_of_zero_tokens_is_a_no_op():
    assert _append(S=0) == _lib.MX_STATUS_OK


def test_python_launch_count_mirrors_the_library_constants():
    """decode.plan()'s "launches" mirrors kMergeFanIn / kMaxMergeItems / kMaxSlots of the
    kernel source."""
    import re
    from mx_flash_attn_kernel_opt__amd import decode
    src = open(os.path.join(REPO, "mx_flash_attn_kernel_opt__amd", "csrc",
                            "paged_decode.hip")).read()
    assert int(re.search(r"kMergeFanIn = (\d+);", src).group(1)) == decode.MERGE_FAN_IN
    assert re.search(r"kMaxMergeItems = 8 \* 8 \* 8 \* 8;", src) and decode.MAX_MERGE_ITEMS == 4096
    m = re.search(r"kMaxSlots = (\d+) \+ (\d+);", src)
    assert int(m.group(1)) + int(m.group(2)) == decode.COUNTER_SLOTS
    assert int(re.search(r"kMaxHandoffBytes = (0x[0-9a-f]+);", src).group(1), 16) == \
        decode.MAX_HANDOFF_BYTES
    assert plan(4, 32, 8, 128, 16, 64, 0, 4, num_cus=256)["launches"] == 1
    assert plan(4, 32, 8, 128, 16, 64, 0, 32, num_cus=256)["launches"] == 1    # two-level tree
    assert plan(1, 32, 8, 128, 16, 4096, 0, 4096, num_cus=256)["launches"] == 1  # 4 levels
    assert plan(1, 32, 8, 128, 16, 8193, 0, 8193, num_cus=256)["launches"] == 2  # > 8^4 splits
    # 193 sequences x 8 KV heads x 8 counter groups (64 splits) exceed the 12 288 counters
    assert plan(193, 32, 8, 128, 16, 64, 0, 64, num_cus=256)["launches"] == 2
    assert plan(192, 32, 8, 128, 16, 64, 0, 64, num_cus=256)["launches"] == 1
    assert plan(64, 32, 8, 128, 16, 64, 0, 0, num_cus=256)["launches"] == 1   # balanced
    # the long-context configurations are one launch
    for B, L in ((1, 32768), (1, 131072), (4, 32768), (4, 131072)):
        assert plan(B, 64, 8, 128, 16, L // 16, 0, 0, num_cus=256)["launches"] == 1


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("SQ", [1, 4, 16])
def test_one_launch_partials_fit_the_handoff_offsets(D, SQ):
    """The in-kernel merges address the fp32 o partials through buffer instructions with 32-bit
    byte offsets: every one-launch split-grid plan keeps them below 2^31 bytes, and so does the
    balanced schedule's whole workspace.  Swept over batches, group sizes and requested split
    counts up to the counter region's limit."""
    from mx_flash_attn_kernel_opt__amd import decode
    seen_one = seen_two = 0
    for B in (1, 7, 64, 512, 4096):
        if B * SQ > 65535:
            continue
        for Hq, Hkv in ((128, 1), (64, 8), (32, 32), (128, 128)):
            for ns in (0, 2, 16, 64, 256, 4096):
                try:
                    p = plan(B, Hq, Hkv, D, 16, 8192, 0, ns, num_cus=256, seqlen_q=SQ)
                except MXAttnError:
                    continue
                o_bytes = B * SQ * Hq * p["splits"] * D * 4
                if p["schedule"].startswith("balanced"):
                    assert p["workspace_bytes"] <= decode.MAX_HANDOFF_BYTES
                elif p["splits"] > 1 and p["launches"] == 1:
                    seen_one += 1
                    assert o_bytes <= decode.MAX_HANDOFF_BYTES, (B, SQ, Hq, Hkv, D, ns, p)
                elif p["splits"] > 1:
                    seen_two += 1
    assert seen_one > 0 and seen_two > 0


@pytest.mark.parametrize("B,SQ,Hq,Hkv,ns,paired", [
    (2, 1, 32, 4, 5, True),      # G = 8: pairs of heads, one 16-row tile
    (2, 2, 32, 4, 5, True),      # 16 rows per head: still paired
    (2, 3, 32, 4, 5, False),     # 24 rows per head: two passes per pair would re-read it
    (2, 1, 12, 3, 5, False),     # odd Hkv
    (2, 1, 64, 2, 20, True),     # G = 32 > 16 rows: not paired
])
def test_fp8_plan_pairs_head_dim_64_heads(B, SQ, Hq, Hkv, ns, paired):
    """At head_dim 64 the fp8 entry runs adjacent KV heads in pairs (one unit of work per pair)
    when a head's query rows fit one 16-row tile; the workspace size covers both formats."""
    if Hq // Hkv * SQ > 16:
        paired = False
    a = plan(B, Hq, Hkv, 64, 16, 64, 0, ns, num_cus=256, seqlen_q=SQ)
    b = plan(B, Hq, Hkv, 64, 16, 64, 0, ns, num_cus=256, seqlen_q=SQ, fp8=True)
    assert b["splits"] == a["splits"] > 1
    assert b["workgroups"] * (2 if paired else 1) == a["workgroups"]
    n = _lib.load().mx_paged_gqa_decode_workspace_size(B, SQ, Hq, Hkv, 64, 16, 64, 0, ns)
    assert n >= max(a["workspace_bytes"], b["workspace_bytes"])
    for D in (128, 256):   # other head dims: the same plan for both formats
        assert (plan(B, Hq, Hkv, D, 16, 64, 0, ns, num_cus=256, seqlen_q=SQ) ==
                plan(B, Hq, Hkv, D, 16, 64, 0, ns, num_cus=256, seqlen_q=SQ, fp8=True))


# ------------------------------------------------------------------------------------------
# Sharded-decode entry points: validation (no HIP call is reached on these paths)
# ------------------------------------------------------------------------------------------

def _partial(**over):
    args = dict(q=FAKE, k=FAKE, v=FAKE, o=FAKE, lse=FAKE, lens=FAKE, table=FAKE, B=2, SQ=1,
                Hq=32, Hkv=8, D=128, P=16, pages=64, max_pages=32, max_seq=0, causal=0,
                scale=0.088, ns=2, ws=FAKE, ws_bytes=1 << 30, stream=None)
    args.update(over)
    a = args
    return _lib.load().mx_paged_gqa_decode_partial(
        a["q"], a["k"], a["v"], a["o"], a["lse"], a["lens"], a["table"], a["B"], a["SQ"],
        a["Hq"], a["Hkv"], a["D"], a["P"], a["pages"], a["max_pages"], a["max_seq"], a["causal"],
        a["scale"], a["ns"], a["ws"], a["ws_bytes"], a["stream"])


@pytest.mark.parametrize("over,status", [
    (dict(o=None), _lib.MX_STATUS_NULL_POINTER),
    (dict(lse=None), _lib.MX_STATUS_NULL_POINTER),
    (dict(table=None), _lib.MX_STATUS_NULL_POINTER),
    (dict(o=ctypes.c_void_p(0x1008)), _lib.MX_STATUS_INVALID_ARGUMENT),   # not 16-byte aligned
    (dict(lse=ctypes.c_void_p(0x1002)), _lib.MX_STATUS_INVALID_ARGUMENT),
    (dict(Hq=30, Hkv=8), _lib.MX_STATUS_INVALID_SHAPE),
    (dict(D=96), _lib.MX_STATUS_UNSUPPORTED),
    (dict(causal=2), _lib.MX_STATUS_INVALID_ARGUMENT),
    (dict(scale=float("nan")), _lib.MX_STATUS_INVALID_ARGUMENT),
    (dict(ws_bytes=100), _lib.MX_STATUS_WORKSPACE_TOO_SMALL),
])
def test_partial_decode_rejects_invalid_arguments(over, status):
    assert _partial(**over) == status
    assert _lib.load().mx_last_error()


def _merge(o=FAKE, lse=FAKE, parts=4, rows=10, D=128, out=FAKE):
    return _lib.load().mx_lse_merge(o, lse, parts, rows, D, out, None)


@pytest.mark.parametrize("over,status", [
    (dict(o=None), _lib.MX_STATUS_NULL_POINTER),
    (dict(lse=None), _lib.MX_STATUS_NULL_POINTER),
    (dict(out=None), _lib.MX_STATUS_NULL_POINTER),
    (dict(parts=0), _lib.MX_STATUS_INVALID_SHAPE),
    (dict(rows=-1), _lib.MX_STATUS_INVALID_SHAPE),
    (dict(D=96), _lib.MX_STATUS_UNSUPPORTED),
    (dict(o=ctypes.c_void_p(0x1008)), _lib.MX_STATUS_INVALID_ARGUMENT),
    (dict(out=ctypes.c_void_p(0x1004)), _lib.MX_STATUS_INVALID_ARGUMENT),
    (dict(rows=(1 << 25) + 1), _lib.MX_STATUS_UNSUPPORTED),
])
def test_lse_merge_rejects_invalid_arguments(over, status):
    assert _merge(**over) == status
    assert _lib.load().mx_last_error()


def test_lse_merge_of_zero_rows_is_a_no_op():
    assert _merge(rows=0) == _lib.MX_STATUS_OK


def test_shard_pages_rejects_bad_arguments():
    import torch
    from mx_flash_attn_kernel_opt__amd import shard_pages
    table = torch.zeros(2, 4, dtype=torch.int32)
    lens = torch.tensor([5, 9], dtype=torch.int32)
    with pytest.raises(ValueError):
        shard_pages(table, lens, 16, 0)
    with pytest.raises(ValueError):
        shard_pages(table, lens, 16, 2, seqlen_q=0)
    with pytest.raises(ValueError):
        shard_pages(table, lens[:1], 16, 2)


def test_balanced_schedule_bounds_its_32_bit_chunk_line():
    """The balanced kernel counts the batch's chunks in 32-bit integers: plans whose units times
    capacity chunks reach 2^30 take the split grid, and forcing the balanced schedule fails."""
    # 512 x 16 units of 4M tokens (262 144 chunks each): 2^31 chunks of capacity
    p = plan(512, 16, 16, 128, 256, 16384, 0, 0, num_cus=256)
    assert p["schedule"] == "split_grid_paired"  # a split grid, over pairs of heads
    with pytest.raises(MXAttnError) as e:
        plan(512, 16, 16, 128, 256, 16384, 0, -10, num_cus=256)
    assert e.value.status == _lib.MX_STATUS_UNSUPPORTED
    # the same batch with a 64K-token capacity stays balanced
    assert plan(512, 16, 16, 128, 256, 16384, 65536, 0,
                num_cus=256)["schedule"] == "balanced_paired"


# ------------------------------------------------------------------------------------------
# Append-and-attend: validation (no HIP call is reached on these paths)
# ------------------------------------------------------------------------------------------

def _decode_append(**over):
    a = dict(q=FAKE, kn=FAKE, vn=FAKE, k=FAKE, v=FAKE, out=FAKE, lens=FAKE, table=FAKE, B=2,
             SQ=1, S=1, Hq=32, Hkv=8, D=128, P=16, pages=64, max_pages=32, max_seq=0, causal=0,
             scale=0.088, ns=2, ws=FAKE, ws_bytes=1 << 30, stream=None)
    a.update(over)
    return _lib.load().mx_paged_gqa_decode_append(
        a["q"], a["kn"], a["vn"], a["k"], a["v"], a["out"], a["lens"], a["table"], a["B"],
        a["SQ"], a["S"], a["Hq"], a["Hkv"], a["D"], a["P"], a["pages"], a["max_pages"],
        a["max_seq"], a["causal"], a["scale"], a["ns"], a["ws"], a["ws_bytes"], a["stream"])


@pytest.mark.parametrize("over,status", [
    (dict(q=None), _lib.MX_STATUS_NULL_POINTER),
    (dict(out=None), _lib.MX_STATUS_NULL_POINTER),
    (dict(kn=None), _lib.MX_STATUS_NULL_POINTER),
    (dict(table=None), _lib.MX_STATUS_NULL_POINTER),
    (dict(vn=ctypes.c_void_p(0x1008)), _lib.MX_STATUS_INVALID_ARGUMENT),
    (dict(q=ctypes.c_void_p(0x1008)), _lib.MX_STATUS_INVALID_ARGUMENT),
    (dict(pages=0), _lib.MX_STATUS_INVALID_SHAPE),          # the pool bounds every write
    (dict(S=-1), _lib.MX_STATUS_INVALID_SHAPE),
    (dict(Hq=30), _lib.MX_STATUS_INVALID_SHAPE),
    (dict(D=96), _lib.MX_STATUS_UNSUPPORTED),
    (dict(causal=3), _lib.MX_STATUS_INVALID_ARGUMENT),
    (dict(ws_bytes=100), _lib.MX_STATUS_WORKSPACE_TOO_SMALL),
])
def test_append_and_attend_rejects_invalid_arguments(over, status):
    assert _decode_append(**over) == status
    assert _lib.load().mx_last_error()


# ------------------------------------------------------------------------------------------
# fp8 K/V cache: validation (no HIP call is reached on these paths)
# ------------------------------------------------------------------------------------------

def _decode_fp8(**over):
    a = dict(q=FAKE, k=FAKE, v=FAKE, out=FAKE, lens=FAKE, table=FAKE, B=2, SQ=1, Hq=32, Hkv=8,
             D=128, P=16, pages=64, max_pages=32, max_seq=0, causal=0, scale=0.088,
             k_scale=0.5, v_scale=2.0, ns=2, ws=FAKE, ws_bytes=1 << 30, phase=0, stream=None)
    a.update(over)
    return _lib.load().mx_paged_gqa_decode_fp8kv(
        a["q"], a["k"], a["v"], a["out"], a["lens"], a["table"], a["B"], a["SQ"], a["Hq"],
        a["Hkv"], a["D"], a["P"], a["pages"], a["max_pages"], a["max_seq"], a["causal"],
        a["scale"], a["k_scale"], a["v_scale"], a["ns"], a["ws"], a["ws_bytes"], a["phase"],
        a["stream"])


@pytest.mark.parametrize("over,status", [
    (dict(q=None), _lib.MX_STATUS_NULL_POINTER),
    (dict(k=None), _lib.MX_STATUS_NULL_POINTER),
    (dict(table=None), _lib.MX_STATUS_NULL_POINTER),
    (dict(k_scale=float("nan")), _lib.MX_STATUS_INVALID_ARGUMENT),
    (dict(v_scale=float("inf")), _lib.MX_STATUS_INVALID_ARGUMENT),
    (dict(scale=1e30, k_scale=1e30), _lib.MX_STATUS_INVALID_ARGUMENT),
    (dict(v=ctypes.c_void_p(0x1008)), _lib.MX_STATUS_INVALID_ARGUMENT),
    (dict(Hq=30), _lib.MX_STATUS_INVALID_SHAPE),
    (dict(D=96), _lib.MX_STATUS_UNSUPPORTED),
    (dict(causal=3), _lib.MX_STATUS_INVALID_ARGUMENT),
    (dict(ws_bytes=100), _lib.MX_STATUS_WORKSPACE_TOO_SMALL),
])
def test_fp8_decode_rejects_invalid_arguments(over, status):
    assert _decode_fp8(**over) == status
    assert _lib.load().mx_last_status() == status
