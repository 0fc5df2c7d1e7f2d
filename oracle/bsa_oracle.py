"""CPU oracle for Mosaic's three-branch block-sparse attention forward.

TEST INFRASTRUCTURE ONLY.  This module is the checker for the HIP implementation in
``mosaic_amd``: only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The product path never calls it and has no CPU fallback.

It restates the reference computation in torch on the CPU, with fp32 accumulation and the
reference's own bf16 rounding points:

  * ``pool_mean``          primitives.py:65-66,76   einops ``reduce(..., 'mean')`` on bf16 -> bf16
  * ``dense_attention``    primitives.py:31,77      flash_attn_func defaults: scale d^-0.5,
                                                    non-causal, GQA head i -> kv head i // G;
                                                    fp32 logits and row sums, P rounded to
                                                    bf16 before P.V, output rounded to bf16
  * ``block_attention``    primitives.py:28-32      attention inside contiguous blocks
  * ``topk_scores``        primitives.py:35-49      repeat_interleave K, bf16 matmul, strided
                                                    '(g h)' mean over query heads (bf16)
  * ``attn_topk``          primitives.py:35-51      topk(largest, sorted) of those scores
  * ``sparse_attn_fwd``    ops.py:41-134, 557-566   selected-branch kernel: q pre-scaled by
                                                    scale*log2(e) and rounded to bf16, exp2
                                                    online softmax in top-k order, P rounded
                                                    to bf16 before PV, LSE in base 2
  * ``mosaic_attn_func``   primitives.py:54-89      branch logic, variants and bf16 merge
  * ``sparse_attn_bwd``    ops.py:179-507           selected-branch backward: grad q over the
                                                    selected blocks, grad k / v over the
                                                    queries whose block selected the key
  * ``sparse_attn_bwd_blocks`` (same lines)         the same for a sample of query and key
                                                    blocks, gathering only selected blocks

Parity pinning (each function is checked against something other than its own formula by
tests/test_oracle.py): einops itself for the strided mean, brute-force masked dense
attention, torch SDPA for dense attention, closed forms for pooling/merge, planted winners
and brute-force argsort for top-k.  ``dense_attention`` restates flash-attn (a third-party
CUDA library, ``flash-attn>=2.0`` unpinned in requirements.txt:9, absent here); it is pinned
against torch's SDPA and a float64 brute force, not bit-wise against flash-attn.
"""

from __future__ import annotations

import torch

LOG2E = 1.44269504089  # ops.py:41


def _check_bnhd(x: torch.Tensor, name: str) -> None:
    if x.dim() != 4:
        raise ValueError(f"{name} must be [B, N, H, d], got {tuple(x.shape)}")


def pool_mean(x: torch.Tensor, block_size: int) -> torch.Tensor:
    """Mean of each run of ``block_size`` tokens: [B, N, H, d] -> [B, N/bs, H, d] (primitives.py:65).

    einops ``reduce(x, 'b (nb bs) h d -> b nb h d', 'mean')`` is ``x.view(...).mean(2)`` on the
    input dtype, i.e. fp32 accumulation and one rounding to the input dtype.
    """
    _check_bnhd(x, "x")
    B, N, H, d = x.shape
    if N % block_size:
        raise ValueError("sequence length must be a multiple of the block size")
    return x.reshape(B, N // block_size, block_size, H, d).mean(dim=2)


def dense_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float | None = None):
    """softmax(q k^T * scale) v with GQA as flash_attn_func computes it, output in q's dtype.

    q [B, T, Hq, d], k/v [B, S, Hk, d]; query head i uses kv head i // (Hq/Hk).  flash-attn's
    published algorithm (primitives.py:31,77 call it with its defaults): fp32 logits, P =
    exp(s - m) in fp32 with m the row maximum, P rounded to the input dtype for the P.V
    product (fp32 accumulate), the fp32 row sum of the unrounded P as the divisor.  flash-attn
    takes m as a running maximum over key tiles; the final row maximum used here gives the
    same rounding error bound per element.
    """
    B, T, Hq, d = q.shape
    Hk = k.shape[2]
    G = Hq // Hk
    scale = d ** -0.5 if scale is None else scale
    qf = q.float().permute(0, 2, 1, 3)                       # B Hq T d
    kf = k.float().repeat_interleave(G, dim=2).permute(0, 2, 3, 1)   # B Hq d S
    vf = v.float().repeat_interleave(G, dim=2).permute(0, 2, 1, 3)   # B Hq S d
    s = torch.matmul(qf, kf) * scale
    p = torch.exp(s - s.amax(dim=-1, keepdim=True))
    o = torch.matmul(p.to(q.dtype).float(), vf) / p.sum(dim=-1, keepdim=True)   # B Hq T d
    return o.permute(0, 2, 1, 3).to(q.dtype)


def block_attention(q, k, v, block_size: int):
    """Attention restricted to contiguous blocks of ``block_size`` tokens (primitives.py:28-32)."""
    B, N, Hq, d = q.shape
    Hk = k.shape[2]
    if N % block_size:
        raise ValueError("sequence length must be a multiple of block_attn_size")
    nb = N // block_size
    qb = q.reshape(B * nb, block_size, Hq, d)
    kb = k.reshape(B * nb, block_size, Hk, d)
    vb = v.reshape(B * nb, block_size, Hk, d)
    return dense_attention(qb, kb, vb).reshape(B, N, Hq, d)


def topk_scores(q_cmp: torch.Tensor, k_cmp: torch.Tensor) -> torch.Tensor:
    """Block-to-block selection scores [B, Hk, nb, nb] (bf16) as attn_topk builds them.

    primitives.py:39 repeats each kv head G times (query head j pairs with kv head j // G);
    :41-44 is an unscaled bf16 matmul; :47 averages query heads with the pattern
    '(g h)' -> h, so row h averages query heads h, h+Hk, h+2Hk, ... (a strided group).
    """
    B, nb, Hq, d = q_cmp.shape
    Hk = k_cmp.shape[2]
    G = Hq // Hk
    k_rep = k_cmp.repeat_interleave(G, dim=2)
    scores = torch.matmul(q_cmp.permute(0, 2, 1, 3), k_rep.permute(0, 2, 3, 1))  # B Hq t u, bf16
    if Hq != Hk:
        scores = scores.reshape(B, G, Hk, nb, nb).mean(dim=1)  # (g h): g is the outer factor
    return scores


def attn_topk(q_cmp: torch.Tensor, k_cmp: torch.Tensor, block_count: int) -> torch.Tensor:
    """Top-``block_count`` key blocks per (batch, query block, kv head): int64 [B, nb, Hk, K]."""
    s = topk_scores(q_cmp, k_cmp).permute(0, 2, 1, 3)  # B t h u  (primitives.py:49)
    return s.topk(k=block_count, dim=-1, largest=True)[1]


def sparse_attn_fwd(q, k, v, block_indices, block_size: int, softmax_scale: float | None = None,
                    q_blocks: torch.Tensor | None = None):
    """Selected-branch forward (ops.py:20-134): returns (o [B,N,Hq,d] in v's dtype, lse fp32).

    For query token n in block i = n // block_size, query head j and kv head c = j // G the
    kernel attends to the tokens of blocks ``block_indices[b, i, c, :]`` in that order with a
    base-2 online softmax.  ``q_blocks`` restricts the computation to a subset of query blocks
    (the other rows of the result are zero); it lets tests check a sample of a large problem.
    """
    _check_bnhd(q, "q")
    B, N, Hq, d = q.shape
    Hk = k.shape[2]
    G = Hq // Hk
    bs = block_size
    nb = N // bs
    K = block_indices.shape[-1]
    scale = d ** -0.5 if softmax_scale is None else softmax_scale
    qsel = torch.arange(nb) if q_blocks is None else torch.as_tensor(q_blocks, dtype=torch.long)
    nq = qsel.numel()

    # ops.py:91-92: q * softmax_scale * LOG2_E in fp32, rounded to bf16
    qs = ((q.float() * scale) * LOG2E).to(torch.bfloat16).float()
    qs = qs.reshape(B, nb, bs, Hk, G, d)[:, qsel].permute(0, 1, 3, 4, 2, 5)   # B nq Hk G bs d
    kb = k.float().reshape(B, nb, bs, Hk, d).permute(0, 3, 1, 2, 4)          # B Hk nb bs d
    vb = v.float().reshape(B, nb, bs, Hk, d).permute(0, 3, 1, 2, 4)
    idx = block_indices.long()[:, qsel]                                        # B nq Hk K

    m = torch.full((B, nq, Hk, G, bs), float("-inf"))
    lsum = torch.zeros((B, nq, Hk, G, bs))
    acc = torch.zeros((B, nq, Hk, G, bs, d))
    bidx = torch.arange(B).view(B, 1, 1)
    hidx = torch.arange(Hk).view(1, 1, Hk)
    for i in range(K):                                    # ops.py:94
        blk = idx[..., i]                                 # B nq Hk
        kt = kb[bidx, hidx, blk]                          # B nq Hk bs d
        vt = vb[bidx, hidx, blk]
        s = torch.matmul(qs, kt.unsqueeze(3).transpose(-1, -2))   # B nq Hk G bs bs (fp32)
        new_max = torch.maximum(m, s.amax(dim=-1))        # ops.py:120-122
        rescale = torch.exp2(m - new_max)                 # ops.py:123
        p = torch.exp2(s - new_max.unsqueeze(-1))         # ops.py:124
        lsum = lsum * rescale + p.sum(dim=-1)             # ops.py:125
        acc = acc * rescale.unsqueeze(-1)                 # ops.py:127
        acc = acc + torch.matmul(p.to(torch.bfloat16).float(), vt.unsqueeze(3))   # ops.py:128
        m = new_max
    o = acc / lsum.unsqueeze(-1)                          # ops.py:130
    lse = m + torch.log2(lsum)                            # ops.py:131

    out = torch.zeros(B, nb, bs, Hk, G, d, dtype=v.dtype)
    out[:, qsel] = o.permute(0, 1, 4, 2, 3, 5).to(v.dtype)
    lse_out = torch.zeros(B, nb, bs, Hk, G)
    lse_out[:, qsel] = lse.permute(0, 1, 4, 2, 3)
    return out.reshape(B, N, Hq, d), lse_out.reshape(B, N, Hq)


LN2 = 0.69314718056   # ops.py:197


def sparse_attn_bwd(q, k, v, o, lse, grad_o, block_indices, block_size: int, softmax_scale: float | None = None):
    """Selected-branch backward (ops.py:179-507): returns (dq, dk, dv) in q's / k's dtype.

    Rounding points of the reference kernels: q' = bf16((q * scale) * log2 e) (ops.py:237,
    412-414); delta = bf16(sum(bf16(o * do))) (ops.py:458, eager bf16 ops); grad q: P =
    exp2(q'.k - lse) * ln2, dS = bf16(P (dP - delta)), dq = bf16((sum dS k * scale) * log2 e)
    (ops.py:265-273); grad k/v over every query whose block selected the key (the block mask,
    ops.py:276-297): P = exp2(k.q' - lse), dv += bf16(P) do, dS = bf16(P (dP - delta) ln2),
    dk += dS q' (ops.py:425-431).  Grad q loops over the index entries (ops.py:244), so a block
    listed twice in a row counts twice there, while the boolean block mask counts it once
    for grad k / v.  Dense N x N masked matrices: for test sizes only.
    """
    B, N, Hq, d = q.shape
    Hk = k.shape[2]
    G = Hq // Hk
    bs = block_size
    nb = N // bs
    scale = d ** -0.5 if softmax_scale is None else softmax_scale
    bf = torch.bfloat16
    qs = ((q.float() * scale) * LOG2E).to(bf).float()
    kf, vf, gf = k.float(), v.float(), grad_o.to(bf).float()
    delta = (o.to(bf) * grad_o.to(bf)).sum(dim=-1).to(bf).float()           # B N Hq
    idx = block_indices.long()
    # mask[b, c, t, u]: query block t selected key block u for kv head c (the block mask)
    count = torch.zeros(B, Hk, nb, nb)
    valid = (idx >= 0) & (idx < nb)
    bb, tt, cc, ii = torch.nonzero(valid, as_tuple=True)
    count.index_put_((bb, cc, tt, idx[bb, tt, cc, ii]), torch.ones(bb.numel()), accumulate=True)
    cnt = count.repeat_interleave(bs, dim=2).repeat_interleave(bs, dim=3)    # B Hk N N entries per key
    tok = cnt > 0                                                            # the block mask
    dq = torch.zeros(B, N, Hq, d)
    dk = torch.zeros(B, N, Hk, d)
    dv = torch.zeros(B, N, Hk, d)
    for b in range(B):
        for j in range(Hq):
            c = j // G
            m = tok[b, c]
            s = qs[b, :, j] @ kf[b, :, c].t()                                   # N x N fp32
            dp = gf[b, :, j] @ vf[b, :, c].t()
            x = torch.where(m, s - lse[b, :, j, None].float(), torch.full_like(s, float("-inf")))
            p = torch.exp2(x)
            dl = delta[b, :, j, None]
            ds_q = (p * LN2 * (dp - dl)).to(bf).float()                         # ops.py:266-269
            dq[b, :, j] = (((ds_q * cnt[b, c]) @ kf[b, :, c]) * scale) * LOG2E  # ops.py:244, 270-272
            dv[b, :, c] += p.to(bf).float().t() @ gf[b, :, j]                   # ops.py:427
            ds_k = (p * (dp - dl) * LN2).to(bf).float()                         # ops.py:429
            dk[b, :, c] += ds_k.t() @ qs[b, :, j]                               # ops.py:430
    return dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype)


def sparse_attn_bwd_blocks(q, k, v, o, lse, grad_o, block_indices, block_size: int, q_blocks, k_blocks,
                           softmax_scale: float | None = None):
    """Selected-branch backward (ops.py:179-507) for a sample of blocks, gathering only the
    selected key blocks, so full-size problems fit: returns (dq rows of the query blocks
    ``q_blocks`` [B, len(q_blocks) * bs, Hq, d], dk and dv rows of the key blocks ``k_blocks``
    [B, len(k_blocks) * bs, Hk, d]), with the arithmetic and rounding points of
    ``sparse_attn_bwd``.  grad q walks the selection entries of each query block in order
    (ops.py:244, duplicates counted); grad k / v walks, per kv head, the query blocks whose
    selection row holds the key block (the boolean block mask, ops.py:276-297, 367-370) in
    ascending order.
    """
    B, N, Hq, d = q.shape
    Hk = k.shape[2]
    G = Hq // Hk
    bs = block_size
    nb = N // bs
    scale = d ** -0.5 if softmax_scale is None else softmax_scale
    bf = torch.bfloat16
    idx = block_indices.long()
    qb, kb = [int(x) for x in q_blocks], [int(x) for x in k_blocks]

    def rows(x, i):
        return x[:, i * bs:(i + 1) * bs].float()

    def qs_rows(i):   # ops.py:237: q' = bf16((q * scale) * log2 e)
        return ((rows(q, i) * scale) * LOG2E).to(bf).float()

    def delta_rows(i):   # ops.py:458: bf16(sum(bf16(o * do)))
        return (o[:, i * bs:(i + 1) * bs].to(bf) * grad_o[:, i * bs:(i + 1) * bs].to(bf)).sum(-1).to(bf).float()

    dq = torch.zeros(B, len(qb) * bs, Hq, d)
    for n, i in enumerate(qb):
        qs, g, dl, ls = qs_rows(i), rows(grad_o.to(bf), i), delta_rows(i), rows(lse, i)
        for b in range(B):
            for j in range(Hq):
                c = j // G
                acc = torch.zeros(bs, d)
                for u in idx[b, i, c].tolist():
                    if not 0 <= u < nb:
                        continue
                    kt, vt = k[b, u * bs:(u + 1) * bs, c].float(), v[b, u * bs:(u + 1) * bs, c].float()
                    p = torch.exp2(qs[b, :, j] @ kt.t() - ls[b, :, j, None])
                    dp = g[b, :, j] @ vt.t()
                    ds = (p * LN2 * (dp - dl[b, :, j, None])).to(bf).float()     # ops.py:266-269
                    acc += ds @ kt
                dq[b, n * bs:(n + 1) * bs, j] = (acc * scale) * LOG2E           # ops.py:270-272
    dk = torch.zeros(B, len(kb) * bs, Hk, d)
    dv = torch.zeros(B, len(kb) * bs, Hk, d)
    for n, u in enumerate(kb):
        for b in range(B):
            for c in range(Hk):
                kt, vt = k[b, u * bs:(u + 1) * bs, c].float(), v[b, u * bs:(u + 1) * bs, c].float()
                for t in (idx[b, :, c] == u).any(-1).nonzero().flatten().tolist():   # ascending
                    qs, g, dl, ls = qs_rows(t)[b], rows(grad_o.to(bf), t)[b], delta_rows(t)[b], rows(lse, t)[b]
                    for j in range(c * G, (c + 1) * G):
                        p = torch.exp2(qs[:, j] @ kt.t() - ls[:, j, None])
                        dp = g[:, j] @ vt.t()
                        dv[b, n * bs:(n + 1) * bs, c] += p.to(bf).float().t() @ g[:, j]          # ops.py:427
                        ds = (p * (dp - dl[:, j, None]) * LN2).to(bf).float()                    # ops.py:429
                        dk[b, n * bs:(n + 1) * bs, c] += ds.t() @ qs[:, j]                       # ops.py:430
    return dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype)


def mosaic_attn_func(q, k, v, weight_ba_cmp_slc, block_attn_size, sparse_block_size,
                     sparse_block_count, block_attn_only, no_compression=False,
                     block_indices=None, return_parts=False):
    """Three-branch forward with the reference's branch logic and bf16 merge (primitives.py:54-89).

    ``block_indices`` (int64 [B, nb, Hk, K]) replaces the oracle's own top-k; parity tests use
    it to evaluate the oracle on the indices the device chose when they differ only by ties.
    With ``return_parts`` a dict of intermediates (branch outputs, indices, scores) is returned.
    """
    parts = {}
    o_ba = block_attention(q, k, v, block_attn_size)
    parts["o_ba"] = o_ba
    if block_attn_only:
        return (o_ba, parts) if return_parts else o_ba

    q_cmp = pool_mean(q, sparse_block_size)
    k_cmp = pool_mean(k, sparse_block_size)
    parts["q_cmp"], parts["k_cmp"] = q_cmp, k_cmp

    def _select():
        parts["scores"] = topk_scores(q_cmp, k_cmp)
        idx = attn_topk(q_cmp, k_cmp, sparse_block_count) if block_indices is None else block_indices
        parts["block_indices"] = idx
        o_slc, _ = sparse_attn_fwd(q, k, v, idx, sparse_block_size)
        parts["o_slc"] = o_slc
        return o_slc

    w = weight_ba_cmp_slc
    if no_compression:                                    # primitives.py:68-74
        o_slc = _select()
        w_ba, w_slc = w[0], w[2]
        w_sum = w_ba + w_slc + 1e-8
        out = o_ba * (w_ba / w_sum) + o_slc * (w_slc / w_sum)
        return (out, parts) if return_parts else out

    v_cmp = pool_mean(v, sparse_block_size)
    o_cmp_blk = dense_attention(q_cmp, k_cmp, v_cmp)       # primitives.py:77
    parts["o_cmp_blk"] = o_cmp_blk
    o_cmp = o_cmp_blk.repeat_interleave(sparse_block_size, dim=1)   # :78

    if sparse_block_count == 0:                           # primitives.py:80-84
        w_ba, w_cmp = w[0], w[1]
        w_sum = w_ba + w_cmp + 1e-8
        out = o_ba * (w_ba / w_sum) + o_cmp * (w_cmp / w_sum)
        return (out, parts) if return_parts else out

    o_slc = _select()
    out = o_ba * w[0] + o_cmp * w[1] + o_slc * w[2]       # primitives.py:89
    return (out, parts) if return_parts else out


def mosaic_attn_func_blocks(q, k, v, weight_ba_cmp_slc, block_attn_size, sparse_block_size,
                            sparse_block_count, q_blocks, block_indices=None):
    """Full-path output (primitives.py:76-89) for the query blocks ``q_blocks`` only.

    Returns (rows [B, len(q_blocks) * sparse_block_size, Hq, d] in q's dtype, parts) where
    parts holds the oracle's selection scores [B, Hk, nb, nb] and the indices used.  The
    pooled tensors, compressed attention and scores are computed for the whole sequence
    (they are small); local and selected attention only for the requested rows.
    """
    B, N, Hq, d = q.shape
    bs, bl = sparse_block_size, block_attn_size
    q_cmp, k_cmp, v_cmp = pool_mean(q, bs), pool_mean(k, bs), pool_mean(v, bs)
    o_cmp_blk = dense_attention(q_cmp, k_cmp, v_cmp)
    scores = topk_scores(q_cmp, k_cmp)
    idx = attn_topk(q_cmp, k_cmp, sparse_block_count) if block_indices is None else block_indices.long().cpu()
    o_slc, _ = sparse_attn_fwd(q, k, v, idx, bs, q_blocks=torch.as_tensor(q_blocks))
    w = weight_ba_cmp_slc
    step = min(bl, bs)
    rows = []
    for i in [int(x) for x in q_blocks]:
        sl = slice(i * bs, (i + 1) * bs)
        o_ba = torch.cat([dense_attention(q[:, t0:t0 + step], k[:, t0 // bl * bl:t0 // bl * bl + bl],
                                          v[:, t0 // bl * bl:t0 // bl * bl + bl])
                          for t0 in range(i * bs, (i + 1) * bs, step)], dim=1)
        o_c = o_cmp_blk[:, i:i + 1].expand(B, bs, Hq, d)
        rows.append(o_ba * w[0][:, sl] + o_c * w[1][:, sl] + o_slc[:, sl] * w[2][:, sl])
    return torch.cat(rows, dim=1), {"scores": scores, "block_indices": idx, "o_cmp_blk": o_cmp_blk}


def selection_band_check(scores_row_major: torch.Tensor, indices: torch.Tensor, block_count: int,
                         band: float = 1e-3):
    """Check device indices against the oracle scores with the tie-band rule.

    ``scores_row_major`` is [B, nb, Hk, nb] (oracle S-bar, any float dtype), ``indices`` the
    device's [B, nb, Hk, K].  With s_K, s_K+1 the K-th and (K+1)-th largest scores of a row,
    every block scoring above s_K+1 + band must be selected, every block scoring below
    s_K - band must not, and the K indices must be distinct and in range.  Returns
    (n_bad_rows, n_ambiguous_rows, n_rows); a row is ambiguous when more blocks lie inside
    the band than there are slots left for them.
    """
    s = scores_row_major.float()
    B, nb, Hk, n = s.shape
    K = block_count
    idx = indices.long()
    if idx.shape != (B, nb, Hk, K):
        raise ValueError(f"indices shape {tuple(idx.shape)} != {(B, nb, Hk, K)}")
    out_of_range = ((idx < 0) | (idx >= n)).any(-1)
    srt = s.sort(dim=-1, descending=True).values
    s_k = srt[..., K - 1]
    s_k1 = srt[..., K] if K < n else torch.full_like(s_k, float("-inf"))
    chosen = torch.zeros_like(s, dtype=torch.bool)
    chosen.scatter_(-1, idx.clamp(0, n - 1), True)
    dup = chosen.sum(-1) != K
    must_in = s > (s_k1 + band).unsqueeze(-1)
    must_out = s < (s_k - band).unsqueeze(-1)
    bad = (must_in & ~chosen).any(-1) | (must_out & chosen).any(-1) | dup | out_of_range
    in_band = ~(must_in | must_out)
    ambiguous = in_band.sum(-1) > (K - must_in.sum(-1))
    return int(bad.sum()), int(ambiguous.sum()), B * nb * Hk


def flops(B, N, Hq, d, block_attn_size, sparse_block_size, block_count):
    """Algorithmic FLOPs of one forward (local + selected + compressed QK^T/PV + top-k scoring)."""
    nb = N // sparse_block_size
    return (4 * B * Hq * d * (N * block_attn_size + N * block_count * sparse_block_size + nb * nb)
            + 2 * B * Hq * d * nb * nb)


def softmax_scale_default(d: int) -> float:
    return d ** -0.5  # ops.py:565


__all__ = [
    "LOG2E", "pool_mean", "dense_attention", "block_attention", "topk_scores", "attn_topk",
    "sparse_attn_fwd", "sparse_attn_bwd", "sparse_attn_bwd_blocks", "mosaic_attn_func", "mosaic_attn_func_blocks",
    "selection_band_check",
    "flops", "softmax_scale_default",
]
