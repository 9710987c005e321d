"""TEST INFRASTRUCTURE ONLY: CPU restatements of the paged GQA decode operator (the checker).

Reference semantics (file:line in the reference tree):
  * math: task.md:138-148 -- kv_head = h // (Hq/Hkv); logits = q . k^T * scale;
    softmax over the valid tokens; out = attn . v;
  * token placement: task.md:94 and :146 -- token t of sequence b is in page
    block_table[b, t // page_size] at offset t % page_size;
  * only the first ceil(L_b / page_size) table entries are valid (task.md:8-10, 61, 92);
  * scale defaults to 1/sqrt(head_dim) (submission_clean.cu:451);
  * multi-token queries: q / out [B, seqlen_q, Hq, D] (task.md:56, 59); with causal
    (task.md:53) query token i sees keys t < L - seqlen_q + i + 1, the end-aligned mask of the
    reference's oracle flash_attn_with_kvcache (verify_real.py:40-41); a query row that sees no
    key is defined as zeros;
  * split ranges and the LSE merge: optimized_c500_flash_attn.cu:537-551 and :666-728,
    submission_c500_regions.py:704-731.
"""

from __future__ import annotations

import math

import numpy as np
import torch


def _as3(q: torch.Tensor) -> torch.Tensor:
    return q.view(q.shape[0], q.shape[2], q.shape[3]) if q.dim() == 4 else q


def kv_bytes(seq_lens, num_kv_heads: int, head_dim: int) -> int:
    """Algorithmic K+V bytes of one call: sum_b L_b * Hkv * D * 2 (K and V) * 2 bytes."""
    total = int(torch.as_tensor(seq_lens).to(torch.int64).clamp(min=0).sum().item())
    return total * num_kv_heads * head_dim * 2 * 2


def _gather_sequence(k_cache, v_cache, block_table, b: int, L: int):
    """Valid K/V rows of sequence b as fp32 [L, Hkv, D] (task.md:94, 146)."""
    P = k_cache.shape[1]
    npg = math.ceil(L / P)
    pages = block_table[b, :npg].to(torch.long)
    k = k_cache.index_select(0, pages).reshape(npg * P, *k_cache.shape[2:])[:L]
    v = v_cache.index_select(0, pages).reshape(npg * P, *v_cache.shape[2:])[:L]
    return k.float(), v.float()


def _visible(L: int, sq: int, causal: bool) -> np.ndarray:
    """[sq, L] bool: key t is visible to query token i (end-aligned causal mask)."""
    t = np.arange(L)[None, :]
    i = np.arange(sq)[:, None]
    return (t < L - sq + i + 1) if causal else np.ones((sq, L), dtype=bool)


def paged_decode_reference(q, k_cache, v_cache, block_table, seq_lens, scale=None,
                           batches=None, causal: bool = False) -> torch.Tensor:
    """fp32 restatement of task.md:138-148 on CPU tensors; returns fp32 of q's shape.

    q is [B, Hq, D] (one query token) or [B, seqlen_q, Hq, D].  One sequence at a time: gather
    its valid pages, upcast to fp32, softmax(q k^T scale) v with query head h reading KV head
    h // group, masked per query token when ``causal``.  Empty sequences (L <= 0) and query
    rows that see no key give zeros.  ``batches`` restricts the computation to some sequences
    (others stay zero).
    """
    q4 = q if q.dim() == 4 else q.unsqueeze(1)
    B, SQ, Hq, D = q4.shape
    Hkv = k_cache.shape[2]
    G = Hq // Hkv
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    lens = torch.as_tensor(seq_lens).cpu()
    out = torch.zeros(B, SQ, Hq, D, dtype=torch.float32)
    for b in (range(B) if batches is None else batches):
        L = int(lens[b])
        if L <= 0:
            continue
        k, v = _gather_sequence(k_cache, v_cache, block_table, b, L)   # [L, Hkv, D]
        qb = q4[b].float().view(SQ, Hkv, G, D).permute(1, 0, 2, 3)     # [Hkv, SQ, G, D]
        qb = qb.reshape(Hkv, SQ * G, D)
        kt = k.permute(1, 2, 0).contiguous()                           # [Hkv, D, L]
        vt = v.permute(1, 0, 2).contiguous()                           # [Hkv, L, D]
        logits = torch.matmul(qb, kt) * scale                          # [Hkv, SQ*G, L]
        vis = torch.from_numpy(np.repeat(_visible(L, SQ, causal), G, axis=0))   # [SQ*G, L]
        logits = logits.masked_fill(~vis, float("-inf"))
        attn = torch.softmax(logits, dim=-1).nan_to_num(0.0)           # no visible key -> 0
        o = torch.matmul(attn, vt)                                     # [Hkv, SQ*G, D]
        out[b] = o.view(Hkv, SQ, G, D).permute(1, 0, 2, 3).reshape(SQ, Hq, D)
    return out if q.dim() == 4 else out[:, 0]


def fp8_dequantize(cache: torch.Tensor, scale: float) -> torch.Tensor:
    """fp32 values of a float8_e4m3fn cache (OCP e4m3fn, torch's conversion) times its
    per-tensor scale."""
    assert cache.dtype == torch.float8_e4m3fn
    return cache.float() * float(scale)


def fp8_quantize(x: torch.Tensor, scale: float) -> torch.Tensor:
    """float8_e4m3fn values of x / scale (fp32 quotient), saturated to [-448, 448] (NaN stays
    NaN) and rounded to nearest, ties to even (torch's conversion): what an append into a
    per-tensor-scaled fp8 cache stores."""
    v = x.float() / torch.tensor(float(scale), dtype=torch.float32)
    v = torch.where(v > 448.0, torch.full_like(v, 448.0),
                    torch.where(v < -448.0, torch.full_like(v, -448.0), v))
    return v.to(torch.float8_e4m3fn)


def paged_decode_fp8_reference(q, k_cache, v_cache, block_table, seq_lens, scale=None,
                               k_scale: float = 1.0, v_scale: float = 1.0,
                               causal: bool = False) -> torch.Tensor:
    """The decode over an fp8 K/V cache: paged_decode_reference on the dequantized caches
    (keys k_scale times the stored e4m3fn values, values v_scale times theirs), the semantics
    of a per-tensor-scaled fp8 KV cache."""
    return paged_decode_reference(q, fp8_dequantize(k_cache, k_scale),
                                  fp8_dequantize(v_cache, v_scale), block_table, seq_lens,
                                  scale, causal=causal)


def paged_decode_fp64(q, k_cache, v_cache, block_table, seq_lens, scale=None,
                      causal: bool = False) -> np.ndarray:
    """fp64 numpy brute force, token by token (tiny shapes only).  Returns q's shape:
    [B, Hq, D] or [B, seqlen_q, Hq, D]; query token i of seqlen_q sees keys
    t < L - seqlen_q + i + 1 when ``causal``, and a row with no visible key is zeros."""
    qt = torch.as_tensor(q)
    q4 = qt if qt.dim() == 4 else qt.unsqueeze(1)
    qn = q4.float().numpy().astype(np.float64)
    kn = torch.as_tensor(k_cache).float().numpy().astype(np.float64)
    vn = torch.as_tensor(v_cache).float().numpy().astype(np.float64)
    bt = torch.as_tensor(block_table).numpy()
    lens = torch.as_tensor(seq_lens).numpy()
    B, SQ, Hq, D = qn.shape
    P, Hkv = kn.shape[1], kn.shape[2]
    G = Hq // Hkv
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    out = np.zeros((B, SQ, Hq, D), dtype=np.float64)
    for b in range(B):
        L = int(lens[b])
        for i in range(SQ):
            n_vis = min(L, L - SQ + i + 1) if causal else L
            if n_vis <= 0:
                continue
            for h in range(Hq):
                kvh = h // G
                logits = np.empty(n_vis)
                for t in range(n_vis):
                    page, off = int(bt[b, t // P]), t % P
                    logits[t] = float(np.dot(qn[b, i, h], kn[page, off, kvh])) * scale
                w = np.exp(logits - logits.max())
                w /= w.sum()
                acc = np.zeros(D)
                for t in range(n_vis):
                    page, off = int(bt[b, t // P]), t % P
                    acc += w[t] * vn[page, off, kvh]
                out[b, i, h] = acc
    return out if qt.dim() == 4 else out[:, 0]


def split_partials(q, k_cache, v_cache, block_table, seq_lens, tokens_per_split: int,
                   scale=None):
    """Per-split normalised partial outputs and natural-log LSEs.

    Split s of sequence b covers tokens [s*tps, min((s+1)*tps, L_b)) (page-aligned ranges as
    submission_clean.cu:456-461 / optimized_c500_flash_attn.cu:537-551).  Returns
    (o [B, Hq, ns, D] fp64, lse [B, Hq, ns] fp64, nsv [B]) with empty splits left at
    o = 0, lse = -inf.
    """
    q3 = _as3(q)
    B, Hq, D = q3.shape
    Hkv = k_cache.shape[2]
    G = Hq // Hkv
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    lens = torch.as_tensor(seq_lens).cpu()
    ns = max(1, max(math.ceil(max(int(L), 0) / tokens_per_split) for L in lens))
    o = np.zeros((B, Hq, ns, D))
    lse = np.full((B, Hq, ns), -np.inf)
    nsv = np.zeros(B, dtype=np.int64)
    for b in range(B):
        L = int(lens[b])
        if L <= 0:
            continue
        k, v = _gather_sequence(k_cache, v_cache, block_table, b, L)
        k = k.double().permute(1, 0, 2)   # [Hkv, L, D]
        v = v.double().permute(1, 0, 2)
        qb = q3[b].double().view(Hkv, G, D)
        logits = torch.matmul(qb, k.transpose(1, 2)) * scale   # [Hkv, G, L]
        nsv[b] = math.ceil(L / tokens_per_split)
        for s in range(nsv[b]):
            t0, t1 = s * tokens_per_split, min((s + 1) * tokens_per_split, L)
            x = logits[:, :, t0:t1]
            m = x.max(dim=-1, keepdim=True).values
            p = torch.exp(x - m)
            lsum = p.sum(-1, keepdim=True)
            part = torch.matmul(p, v[:, t0:t1]) / lsum                # [Hkv, G, D]
            o[b, :, s] = part.reshape(Hq, D).numpy()
            lse[b, :, s] = (m + torch.log(lsum)).reshape(Hq).numpy()
    return o, lse, nsv


def combine_partials(o: np.ndarray, lse: np.ndarray, nsv) -> np.ndarray:
    """LSE merge of split partials (optimized_c500_flash_attn.cu:681-727): with
    M = max_s lse_s over the valid splits, out = sum_s e^(lse_s - M) o_s / sum_s e^(lse_s - M)."""
    B, Hq, _, D = o.shape
    out = np.zeros((B, Hq, D))
    for b in range(B):
        n = int(nsv[b])
        if n <= 0:
            continue
        m = lse[b, :, :n].max(axis=-1, keepdims=True)
        w = np.exp(lse[b, :, :n] - m)                              # [Hq, n]
        out[b] = (w[:, :, None] * o[b, :, :n]).sum(1) / w.sum(-1, keepdims=True)
    return out


def paged_kv_append_reference(k_new, v_new, k_cache, v_cache, block_table, seq_lens,
                              k_scale: float = 1.0, v_scale: float = 1.0):
    """Paged K/V append on CPU copies (flash_attn_with_kvcache's k / v arguments; the reference's
    harness passes them as None, verify_real.py:40-41): token j of sequence b is stored at
    position pos = max(L_b, 0) + j, page block_table[b, pos // P], offset pos % P
    (task.md:94, 146).  Slots past the table row or with a page id outside the pool are
    skipped.  float8_e4m3fn caches store fp8_quantize(x, k_scale) / (x, v_scale).  Returns
    (k_cache, v_cache, flags) with flags a set of {"seq_too_long", "bad_page"}."""
    k_out, v_out = k_cache.clone(), v_cache.clone()
    kn = k_new if k_new.dim() == 4 else k_new.unsqueeze(1)
    vn = v_new if v_new.dim() == 4 else v_new.unsqueeze(1)
    if k_cache.dtype == torch.float8_e4m3fn:  # bytes in, bytes out
        kn, vn = fp8_quantize(kn, k_scale).view(torch.uint8), fp8_quantize(vn, v_scale).view(
            torch.uint8)
        k_out, v_out = k_out.view(torch.uint8), v_out.view(torch.uint8)
    B, S = kn.shape[0], kn.shape[1]
    num_pages, P = k_cache.shape[0], k_cache.shape[1]
    width = block_table.shape[1]
    lens = torch.as_tensor(seq_lens).cpu()
    flags = set()
    for b in range(B):
        for j in range(S):
            pos = max(int(lens[b]), 0) + j
            if pos >= width * P:
                flags.add("seq_too_long")
                continue
            pid = int(block_table[b, pos // P])
            if not 0 <= pid < num_pages:
                flags.add("bad_page")
                continue
            k_out[pid, pos % P] = kn[b, j]
            v_out[pid, pos % P] = vn[b, j]
    if k_cache.dtype == torch.float8_e4m3fn:
        k_out, v_out = k_out.view(torch.float8_e4m3fn), v_out.view(torch.float8_e4m3fn)
    return k_out, v_out, flags



def paged_decode_partial_reference(q, k_cache, v_cache, block_table, seq_lens, scale=None,
                                   causal: bool = False):
    """One shard's unmerged decode (the split phase of optimized_c500_flash_attn.cu:537-551 for
    a caller-chosen key range), fp64 on CPU.

    ``block_table`` / ``seq_lens`` describe the shard's keys.  Returns (o, lse): o of q's shape,
    each row's softmax-weighted V over the shard's visible keys; lse of q's shape without D,
    log(sum_t exp(scale * q . k_t)) over them (natural log).  With ``causal`` the end-aligned
    mask is taken on the shard's own length.  Rows that see no key: o = 0, lse = -inf.
    """
    q4 = q if q.dim() == 4 else q.unsqueeze(1)
    B, SQ, Hq, D = q4.shape
    Hkv = k_cache.shape[2]
    G = Hq // Hkv
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    lens = torch.as_tensor(seq_lens).cpu()
    o = torch.zeros(B, SQ, Hq, D, dtype=torch.float64)
    lse = torch.full((B, SQ, Hq), float("-inf"), dtype=torch.float64)
    for b in range(B):
        L = int(lens[b])
        if L <= 0:
            continue
        k, v = _gather_sequence(k_cache, v_cache, block_table, b, L)
        kt = k.double().permute(1, 2, 0)                                # [Hkv, D, L]
        vt = v.double().permute(1, 0, 2)                                # [Hkv, L, D]
        qb = q4[b].double().view(SQ, Hkv, G, D).permute(1, 0, 2, 3).reshape(Hkv, SQ * G, D)
        logits = torch.matmul(qb, kt) * scale                          # [Hkv, SQ*G, L]
        vis = torch.from_numpy(np.repeat(_visible(L, SQ, causal), G, axis=0))
        logits = logits.masked_fill(~vis, float("-inf"))
        lse_b = torch.logsumexp(logits, dim=-1)                        # -inf: no visible key
        attn = torch.exp(logits - lse_b.unsqueeze(-1)).nan_to_num(0.0)
        ob = torch.matmul(attn, vt)                                    # [Hkv, SQ*G, D]
        o[b] = ob.view(Hkv, SQ, G, D).permute(1, 0, 2, 3).reshape(SQ, Hq, D)
        lse[b] = lse_b.view(Hkv, SQ, G).permute(1, 0, 2).reshape(SQ, Hq)
    if q.dim() == 3:
        return o[:, 0], lse[:, 0]
    return o, lse


def lse_merge_reference(o_parts, lse_parts) -> np.ndarray:
    """Log-sum-exp merge of gathered partials (combine_splits, optimized_c500_flash_attn.cu:
    666-728), fp64: o_parts [parts, ..., D], lse_parts [parts, ...] (natural log).  With
    M = max_p lse_p: out = sum_p e^(lse_p - M) o_p / sum_p e^(lse_p - M); rows whose every lse is
    -inf are zeros."""
    o = np.asarray(o_parts, dtype=np.float64)
    ls = np.asarray(lse_parts, dtype=np.float64)
    m = ls.max(axis=0)
    seen = np.isfinite(m)
    w = np.exp(ls - np.where(seen, m, 0.0)[None])                      # 0 for -inf parts
    num = (w[..., None] * o).sum(0)
    den = w.sum(0)
    return np.where(seen[..., None], num / np.where(seen, den, 1.0)[..., None], 0.0)


def paged_decode_append_reference(q, k_new, v_new, k_cache, v_cache, block_table, seq_lens,
                                  scale=None, causal: bool = False):
    """Append-and-attend (flash_attn_with_kvcache with k / v given): the append of
    ``paged_kv_append_reference``, then ``paged_decode_reference`` over max(L_b, 0) + S keys.
    Returns (out fp32 of q's shape, k_cache, v_cache, flags); meaningful when no flag is
    raised (every new token found a slot)."""
    k2, v2, flags = paged_kv_append_reference(k_new, v_new, k_cache, v_cache, block_table,
                                              seq_lens)
    S = k_new.shape[1] if k_new.dim() == 4 else 1
    lens = torch.as_tensor(seq_lens).cpu().to(torch.int32).clamp(min=0) + S
    out = paged_decode_reference(q, k2, v2, block_table, lens, scale, causal=causal)
    return out, k2, v2, flags
