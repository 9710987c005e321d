"""TEST INFRASTRUCTURE ONLY: CPU restatements of the paged GQA decode operator (the checker).

Reference semantics (file:line in the reference tree):
  * math: task.md:138-148 -- kv_head = h // (Hq/Hkv); logits = q . k^T * scale;
    softmax over the valid tokens; out = attn . v;
  * token placement: task.md:94 and :146 -- token t of sequence b is in page
    block_table[b, t // page_size] at offset t % page_size;
  * only the first ceil(L_b / page_size) table entries are valid (task.md:8-10, 61, 92);
  * scale defaults to 1/sqrt(head_dim) (submission_clean.cu:451);
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
    """Algorithmic K+V bytes of one call (BASELINE.md byte formula)."""
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


def paged_decode_reference(q, k_cache, v_cache, block_table, seq_lens, scale=None,
                           batches=None) -> torch.Tensor:
    """fp32 restatement of task.md:138-148 on CPU tensors; returns fp32 [B, Hq, D].

    One sequence at a time: gather its valid pages, upcast to fp32, softmax(q k^T scale) v with
    query head h reading KV head h // group.  Empty sequences (L <= 0) give zeros.
    ``batches`` restricts the computation to some sequences (others stay zero).
    """
    q3 = _as3(q)
    B, Hq, D = q3.shape
    Hkv = k_cache.shape[2]
    G = Hq // Hkv
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    lens = torch.as_tensor(seq_lens).cpu()
    out = torch.zeros(B, Hq, D, dtype=torch.float32)
    for b in (range(B) if batches is None else batches):
        L = int(lens[b])
        if L <= 0:
            continue
        k, v = _gather_sequence(k_cache, v_cache, block_table, b, L)   # [L, Hkv, D]
        qb = q3[b].float().view(Hkv, G, D)                             # [Hkv, G, D]
        kt = k.permute(1, 2, 0).contiguous()                           # [Hkv, D, L]
        vt = v.permute(1, 0, 2).contiguous()                           # [Hkv, L, D]
        logits = torch.matmul(qb, kt) * scale                          # [Hkv, G, L]
        attn = torch.softmax(logits, dim=-1)
        out[b] = torch.matmul(attn, vt).reshape(Hq, D)
    return out


def paged_decode_fp64(q, k_cache, v_cache, block_table, seq_lens, scale=None) -> np.ndarray:
    """fp64 numpy brute force, token by token (tiny shapes only).  Returns [B, Hq, D]."""
    qn = _as3(torch.as_tensor(q)).float().numpy().astype(np.float64)
    kn = torch.as_tensor(k_cache).float().numpy().astype(np.float64)
    vn = torch.as_tensor(v_cache).float().numpy().astype(np.float64)
    bt = torch.as_tensor(block_table).numpy()
    lens = torch.as_tensor(seq_lens).numpy()
    B, Hq, D = qn.shape
    P, Hkv = kn.shape[1], kn.shape[2]
    G = Hq // Hkv
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    out = np.zeros((B, Hq, D), dtype=np.float64)
    for b in range(B):
        L = int(lens[b])
        if L <= 0:
            continue
        for h in range(Hq):
            kvh = h // G
            logits = np.empty(L)
            for t in range(L):
                page, off = int(bt[b, t // P]), t % P
                logits[t] = float(np.dot(qn[b, h], kn[page, off, kvh])) * scale
            w = np.exp(logits - logits.max())
            w /= w.sum()
            acc = np.zeros(D)
            for t in range(L):
                page, off = int(bt[b, t // P]), t % P
                acc += w[t] * vn[page, off, kvh]
            out[b, h] = acc
    return out


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
