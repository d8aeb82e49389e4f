"""fp32 CPU restatement of the reference's prefill and decode attention maths.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""
from __future__ import annotations

import math

import torch

NEG_CLAMP = -1.0e9  # src/flash_attn.py:53-60, src/flash_decode.py:97-99


def _f(t: torch.Tensor, dtype=torch.float32) -> torch.Tensor:
    return t.detach().to("cpu", dtype)


def prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
            sm_scale: float | None = None, dtype=torch.float32):
    """Causal GQA prefill attention -> (out [B,Hq,S,D], lse [B,Hq,S]).

    Follows src/flash_attn.py:85-111 (GQA: query head h reads kv head h // G,
    :92-94) and the kernel src/flash_attn.py:42-83: scores = q.k / sqrt(D)
    (:52), query row i attends keys 0..i, keys are bounded by the query length
    S (:43-44, :55 use seq_len of q), masked scores -1e9 (:53-55).  out is the
    softmax-weighted sum of V; lse = log(sum exp(scores)) over the visible keys
    (natural log of the scaled scores — the extra output this build adds).
    """
    B, Hq, S, D = q.shape
    _, Hkv, L, _ = k.shape
    if L < S:
        raise ValueError("prefill oracle needs at least S keys")
    G = Hq // Hkv
    scale = (1.0 / math.sqrt(D)) if sm_scale is None else sm_scale
    qf = _f(q, dtype)
    kf = _f(k[:, :, :S], dtype).repeat_interleave(G, dim=1)
    vf = _f(v[:, :, :S], dtype).repeat_interleave(G, dim=1)
    scores = torch.matmul(qf, kf.transpose(-1, -2)) * scale
    causal = torch.ones(S, S, dtype=torch.bool).triu(1)
    scores = scores.masked_fill(causal, float("-inf"))
    lse = torch.logsumexp(scores, dim=-1)
    p = torch.exp(scores - lse[..., None])
    out = torch.matmul(p, vf)
    return out, lse


def _valid_keys(B: int, L: int, mask: torch.Tensor | None,
                seq_lens: torch.Tensor | None) -> torch.Tensor:
    """[B, L] bool: key j of batch b participates.

    src/flash_decode.py:85-95 (j < kv_len and mask), mask shapes [L], [B|1, L]
    and [B|1, 1, 1, L] with L' >= L (src/flash_decode.py:215-233); seq_lens is
    this build's graph-safe extension (j < seq_lens[b]).
    """
    valid = torch.ones(B, L, dtype=torch.bool)
    if mask is not None:
        m = mask.detach().to("cpu")
        if m.ndim == 1:
            m = m[:L].expand(B, L)
        else:
            m = m.reshape(m.shape[0], m.shape[-1])[:, :L].expand(B, L)
        valid &= m
    if seq_lens is not None:
        sl = seq_lens.detach().to("cpu", torch.int64)
        valid &= torch.arange(L)[None, :] < sl[:, None]
    return valid


def decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
           mask: torch.Tensor | None = None,
           seq_lens: torch.Tensor | None = None,
           empty: str = "zero", sm_scale: float | None = None,
           dtype=torch.float32):
    """Single-token GQA decode -> (out [B,Hq,1,D], lse [B,Hq]).

    Semantics of flash_decode (src/flash_decode.py:236-370): score_j =
    sum_d k.q * (1/sqrt(D)) (:84, :335), non-participating keys excluded, and a
    row with no participating key gives out = 0 (:204-205) — or NaN when
    empty == "nan", the 0/0 of the legacy decode_attention (src/decode_attn.py:70).
    """
    B, Hq, S, D = q.shape
    _, Hkv, L, _ = k.shape
    G = Hq // Hkv
    scale = (1.0 / math.sqrt(D)) if sm_scale is None else sm_scale
    qf = _f(q[:, :, :1], dtype)
    kf = _f(k, dtype).repeat_interleave(G, dim=1)
    vf = _f(v, dtype).repeat_interleave(G, dim=1)
    valid = _valid_keys(B, L, mask, seq_lens)                       # [B, L]
    if seq_lens is not None:
        # slots at or beyond seq_lens[b] are never read: they contribute
        # nothing even if they hold NaN (masked in-range slots still do 0*v,
        # as in the reference's sum(p * v) at src/flash_decode.py:111)
        in_range = _valid_keys(B, L, None, seq_lens)[:, None, :, None]
        kf = torch.where(in_range, kf, torch.zeros_like(kf))
        vf = torch.where(in_range, vf, torch.zeros_like(vf))
    scores = torch.matmul(qf, kf.transpose(-1, -2))[:, :, 0] * scale  # [B,Hq,L]
    scores = scores.masked_fill(~valid[:, None, :], float("-inf"))
    lse = torch.logsumexp(scores, dim=-1)                             # [B,Hq]
    empty_row = ~valid.any(dim=1)                                     # [B]
    p = torch.exp(scores - lse[..., None])
    p = torch.where(empty_row[:, None, None], torch.zeros_like(p), p)
    out = torch.matmul(p[:, :, None, :], vf)                          # [B,Hq,1,D]
    fill = 0.0 if empty == "zero" else float("nan")
    out = torch.where(empty_row[:, None, None, None], torch.full_like(out, fill), out)
    lse = torch.where(empty_row[:, None], torch.full_like(lse, float("-inf")), lse)
    return out, lse


def split_partials(q, k, v, split_len: int, mask=None, seq_lens=None,
                   block: int = 64, sm_scale: float | None = None):
    """Per-split online-softmax state, as _flash_decode_split_kernel builds it.

    src/flash_decode.py:67-113: for each (b, h, split) keys are visited in
    blocks of `block`; invalid keys score -inf; m_blk = max(max(scores), -1e9);
    alpha = exp(m - m_new); acc = alpha*acc + sum p*v; l = alpha*l + sum p.
    Returns (m, l, acc) with shapes [B,Hq,S], [B,Hq,S], [B,Hq,S,D] (natural-log
    max, clamped at -1e9; an empty split keeps l = 0, acc = 0).
    """
    B, Hq, _, D = q.shape
    _, Hkv, L, _ = k.shape
    G = Hq // Hkv
    scale = (1.0 / math.sqrt(D)) if sm_scale is None else sm_scale
    nsplit = -(-L // split_len)
    valid = _valid_keys(B, L, mask, seq_lens)
    qf = _f(q[:, :, 0])                               # [B,Hq,D]
    kf = _f(k).repeat_interleave(G, dim=1)            # [B,Hq,L,D]
    vf = _f(v).repeat_interleave(G, dim=1)
    m_out = torch.empty(B, Hq, nsplit)
    l_out = torch.empty(B, Hq, nsplit)
    acc_out = torch.empty(B, Hq, nsplit, D)
    all_scores = torch.einsum("bhd,bhld->bhl", qf, kf) * scale
    all_scores = all_scores.masked_fill(~valid[:, None, :], float("-inf"))
    for s in range(nsplit):
        m = torch.full((B, Hq), float("-inf"))
        l = torch.zeros(B, Hq)
        acc = torch.zeros(B, Hq, D)
        for b0 in range(s * split_len, min((s + 1) * split_len, L), block):
            b1 = min(b0 + block, (s + 1) * split_len, L)
            sc = all_scores[:, :, b0:b1]
            m_blk = torch.clamp(sc.max(dim=-1).values, min=NEG_CLAMP)
            m_new = torch.maximum(m, m_blk)
            alpha = torch.exp(m - m_new)
            p = torch.exp(sc - m_new[..., None])
            acc = acc * alpha[..., None] + torch.einsum("bhl,bhld->bhd", p, vf[:, :, b0:b1])
            l = l * alpha + p.sum(-1)
            m = m_new
        m_out[:, :, s] = m
        l_out[:, :, s] = l
        acc_out[:, :, s] = acc
    return m_out, l_out, acc_out


def combine(m: torch.Tensor, l: torch.Tensor, acc: torch.Tensor,
            empty: str = "zero"):
    """LSE combine of split partials (src/flash_decode.py:182-205).

    M = max over splits with l > 0 (clamped at -1e9); w_s = exp(m_s - M) for
    l_s > 0 else 0; den = sum w_s l_s; out = num / max(den, 1) if den > 0 else 0.
    Also returns lse = M + log(den) (-inf for empty rows).
    """
    has = l > 0
    M = torch.where(has, m, torch.full_like(m, float("-inf"))).max(dim=-1).values
    M = torch.clamp(M, min=NEG_CLAMP)
    w = torch.where(has, torch.exp(m - M[..., None]), torch.zeros_like(m))
    den = (w * l).sum(-1)
    num = (w[..., None] * acc).sum(-2)
    fill = 0.0 if empty == "zero" else float("nan")
    out = torch.where(den[..., None] > 0, num / torch.clamp(den, min=1.0)[..., None],
                      torch.full_like(num, fill))
    lse = torch.where(den > 0, M + torch.log(den), torch.full_like(den, float("-inf")))
    return out[:, :, None, :], lse
