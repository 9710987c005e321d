"""MI355X (gfx950) paged GQA decode attention.

The one operator of the reference (task.md:138-148) as a hand-written HIP library,
libmxattn.so, with the reference's C entry point ``run_kernel`` (task.md:38-54) and an
extended C ABI (include/mx_paged_decode.h).  This package loads the library with ctypes and
exposes it over PyTorch-ROCm device tensors; it has no CPU fallback.
"""

from ._lib import MXAttnError, library_path, load  # noqa: F401
from .decode import (  # noqa: F401
    BoundDecode,
    BoundDecodeAppend,
    lse_merge,
    make_workspace,
    paged_gqa_decode,
    paged_gqa_decode_append,
    paged_gqa_decode_partial,
    paged_kv_append,
    plan,
    read_device_status,
    run_kernel,
    workspace_size,
)
from .shard import shard_pages  # noqa: F401

__all__ = [
    "BoundDecode",
    "BoundDecodeAppend",
    "MXAttnError",
    "library_path",
    "load",
    "lse_merge",
    "make_workspace",
    "paged_gqa_decode",
    "paged_gqa_decode_append",
    "paged_gqa_decode_partial",
    "paged_kv_append",
    "plan",
    "read_device_status",
    "run_kernel",
    "shard_pages",
    "workspace_size",
]
