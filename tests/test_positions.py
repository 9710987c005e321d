"""Host check of the append-position arithmetic the kernels use (csrc/positions.h).

seq_lens are int32 and may sit anywhere up to 2^31 - 1; the device code must never form
max(L, 0) + j when that would wrap.  The helpers are compiled here into a small host program
(hipcc, no GPU needed) and compared with the same quantities in unbounded Python integers:
  append_position(L, j, T)  = max(L, 0) + j if that is < T, else -1
  keys_after_append(L, a)   = min(max(L, 0) + a, 2^31 - 1)
"""

from __future__ import annotations

import itertools
import os
import shutil
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(REPO, "mx_flash_attn_kernel_opt__amd", "csrc")
INT32_MAX = 2**31 - 1

PROGRAM = r"""
#include "positions.h"
#include <cstdio>
int main() {
  char op;
  long long a, b, c;
  while (std::scanf(" %c %lld %lld %lld", &op, &a, &b, &c) == 4) {
    if (op == 'p') std::printf("%d\n", append_position((int)a, (int)b, (int)c));
    else std::printf("%d\n", keys_after_append((int)a, (int)b));
  }
  return 0;
}
"""


def _hipcc():
    cand = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc")
    return cand if os.path.exists(cand) else shutil.which("hipcc")


@pytest.fixture(scope="module")
def program(tmp_path_factory):
    hipcc = _hipcc()
    if hipcc is None:
        pytest.skip("hipcc not available")
    d = tmp_path_factory.mktemp("positions")
    src = d / "positions_check.hip"
    src.write_text(PROGRAM)
    exe = d / "positions_check"
    subprocess.run([hipcc, "--offload-arch=gfx950", "-O2", f"-I{CSRC}", str(src), "-o", str(exe)],
                   check=True, capture_output=True)
    return str(exe)


def _run(exe, queries):
    text = "".join(f"{op} {a} {b} {c}\n" for op, a, b, c in queries)
    out = subprocess.run([exe], input=text, capture_output=True, text=True, check=True).stdout
    return [int(x) for x in out.split()]


LENS = [-INT32_MAX - 1, -5, -1, 0, 1, 15, 16, 1000, 2**30, INT32_MAX - 17, INT32_MAX - 16,
        INT32_MAX - 2, INT32_MAX - 1, INT32_MAX]


def test_append_position_never_wraps(program):
    tables = [16, 64, 4096, INT32_MAX - 16, INT32_MAX]
    js = [0, 1, 2, 15, 16, 17, 2**30 - 1]
    queries = [("p", L, j, T) for L, j, T in itertools.product(LENS, js, tables)]
    got = _run(program, queries)
    for (_, L, j, T), g in zip(queries, got):
        pos = max(L, 0) + j
        assert g == (pos if pos < T else -1), (L, j, T, g)


def test_keys_after_append_saturates(program):
    queries = [("k", L, a, 0) for L, a in itertools.product(LENS, [0, 1, 16, 17, 2**30 - 1])]
    got = _run(program, queries)
    for (_, L, a, _), g in zip(queries, got):
        assert g == min(max(L, 0) + a, INT32_MAX), (L, a, g)
