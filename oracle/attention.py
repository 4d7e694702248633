"""CPU oracle for the Flash-HOG attention path (numpy, float64).

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module, and only to check results or as the
timed CPU baseline; the product path never calls it.

It restates the reference's equations with a materialised (N_Q, N_K) score
matrix, one (batch, head) at a time:

  attn_fwd            flash_hog/_jax_refs/jax_impl.py:112-139 (attn_fwd) and the
                      logsumexp residual L of jax_impl.py:423 (jax.nn.logsumexp(S))
  attn_bwd            flash_hog/_jax_refs/jax_impl.py:142-191 (attn_bwd)
  attn_bwd_bwd_stats  flash_hog/_jax_refs/jax_impl.py:273-336 (attn_bwd_bwd_stats),
                      plus the pass statistics D, dD, B of
                      flash_hog/jax/_pallas_gpu_kernel.py:110, :168, :209-210

Layouts follow the reference's seam: q, k, v and friends are (B, T, H, D)
arrays, L is (B, H, T). `causal` is False/0 (no mask), True/1 (top-left: key j
visible to query i iff j <= i, flash_hog/jax/_pallas_gpu_kernel.py:37-41) or 2
(bottom-right: j <= i + N_K - N_Q, jax_impl.py:104-109 get_mask_bottom_right
with an infinite window); the two agree whenever N_Q == N_K. A query that sees
no key (bottom-right, N_Q > N_K) gets O = 0, L = +inf and zero gradients; the
reference's softmax leaves such rows undefined (NaN).

Grouped-query attention: k, v, ddk, ddv may have fewer heads than q (a
divisor); query head h uses key/value head h // (H_q / H_kv), the grouping
"(kv_heads group)" of _pallas_gpu_kernel.py:106-107, and the key-side
gradients sum over the heads of a group (_pallas_gpu_kernel.py:333-370).

How each function is pinned (tests/test_oracle.py):
  attn_fwd            torch.nn.functional.scaled_dot_product_attention and
                      torch.logsumexp (library routines), including its
                      enable_gqa head grouping and its bottom-right causal bias
                      (torch.nn.attention.bias.causal_lower_right); row sums of
                      P == 1; causal row 0 reproduces V_0.
  attn_bwd            torch autograd of textbook attention (fp64); sum over keys
                      of dK == 0.
  attn_bwd_bwd_stats  the reference's golden vectors (test_data.zip);
                      central finite differences of attn_bwd; torch autograd
                      double backward (fp64); sum over keys of dK2 and dV2 == 0;
                      the ddQ = ddK = 0 special case reducing to a first-order
                      backward with V := ddV; linearity in (ddQ, ddK, ddV);
                      the causal prefix property.
  row statistics      D against rowsum(P * dP); dD, B against their definitions
                      through the autograd double backward's outputs.
  grouped heads       the outputs equal those of the ungrouped problem with
                      k, v, ddk, ddv repeated per group and the key-side
                      gradients summed over the group; torch autograd (fp64)
                      of SDPA with enable_gqa for the first backward.
  empty rows          rows that see no key contribute nothing: a bottom-right
                      run with N_Q > N_K equals, on its last N_K rows and on
                      every key-side output, the square run of those rows.
"""

from __future__ import annotations

import numpy as np


def _bhtd(x) -> np.ndarray:
    """(B, T, H, D) -> (B, H, T, D) float64 copy."""
    return np.ascontiguousarray(np.transpose(np.asarray(x, dtype=np.float64), (0, 2, 1, 3)))


def _bthd(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(np.transpose(x, (0, 2, 1, 3)))


def causal_mask(n_q: int, n_k: int, causal=1) -> np.ndarray:
    """Boolean (n_q, n_k): key j visible to query i iff j <= i (causal 1,
    top-left) or j <= i + n_k - n_q (causal 2, bottom-right)."""
    off = n_k - n_q if int(causal) == 2 else 0
    return np.arange(n_k)[None, :] <= np.arange(n_q)[:, None] + off


def _scores(q: np.ndarray, k: np.ndarray, scale: float, causal) -> np.ndarray:
    s = scale * (q @ k.T)
    if causal:
        s = np.where(causal_mask(q.shape[0], k.shape[0], causal), s, -np.inf)
    return s


def _probs(q, k, lse, scale, causal):
    s = _scores(q, k, scale, causal)
    return np.exp(s - lse[:, None])  # masked entries and empty rows (L = +inf) give 0


# --------------------------------------------------------------------------
# single (batch, head) kernels on 2-D arrays
# --------------------------------------------------------------------------

def fwd_head(q, k, v, scale, causal):
    """O and natural-log L of one head (jax_impl.py:112-139, :423)."""
    s = _scores(q, k, scale, causal)
    m = np.max(s, axis=-1, keepdims=True)
    empty = np.isneginf(m)  # rows that see no key
    m = np.where(empty, 0.0, m)
    e = np.exp(s - m)
    z = np.sum(e, axis=-1, keepdims=True)
    zs = np.where(empty, 1.0, z)
    lse = np.where(empty, np.inf, m + np.log(zs))[:, 0]
    return (e / zs) @ v, lse


def bwd_head(q, k, v, o, do, lse, scale, causal):
    """dQ, dK, dV of one head (jax_impl.py:142-191), D = rowsum(O * dO)."""
    p = _probs(q, k, lse, scale, causal)
    dp = do @ v.T
    d = np.sum(o * do, axis=-1)
    ds = scale * p * (dp - d[:, None])
    return ds @ k, ds.T @ q, p.T @ do, d


def bwd_bwd_head(q, k, v, o, do, ddq, ddk, ddv, lse, scale, causal):
    """dQ2, dK2, dV2, ddO and the pass statistics D, dD, B of one head.

    Equations of jax_impl.py:301-336 (attn_bwd_bwd_stats); B is the
    rowsum(dP2 * P) that _pallas_gpu_kernel.py:209-210 accumulates.
    """
    p = _probs(q, k, lse, scale, causal)
    dp = do @ v.T
    dds = scale * (ddq @ k.T + q @ ddk.T)
    d = np.sum(o * do, axis=-1)
    dd = np.sum(dds * p, axis=-1)
    dp2 = do @ ddv.T - dp * dd[:, None] - dds * d[:, None] + dp * dds
    b = np.sum(dp2 * p, axis=-1)
    ds = scale * p * (dp - d[:, None])
    ds2 = scale * p * (dp2 - b[:, None])
    ddp = p * (dds - dd[:, None])
    dq2 = ds @ ddk + ds2 @ k
    dk2 = ds.T @ ddq + ds2.T @ q
    dv2 = ddp.T @ do
    ddo = p @ ddv + ddp @ v
    return dq2, dk2, dv2, ddo, d, dd, b


# --------------------------------------------------------------------------
# batched (B, T, H, D) wrappers
# --------------------------------------------------------------------------

def _group(Q: np.ndarray, K: np.ndarray) -> int:
    """Query heads per key/value head of (B, H, T, D) arrays."""
    H, Hk = Q.shape[1], K.shape[1]
    if H % Hk:
        raise ValueError(f"query heads ({H}) must be a multiple of key/value heads ({Hk})")
    return H // Hk


def attn_fwd(q, k, v, scale: float, causal):
    """Returns O (B, T, H, D) and L (B, H, T), float64."""
    Q, K, V = _bhtd(q), _bhtd(k), _bhtd(v)
    B, H, T, _ = Q.shape
    G = _group(Q, K)
    O = np.empty((B, H, T, V.shape[-1]))
    L = np.empty((B, H, T))
    for b in range(B):
        for h in range(H):
            O[b, h], L[b, h] = fwd_head(Q[b, h], K[b, h // G], V[b, h // G], scale, causal)
    return _bthd(O), L


def attn_bwd(q, k, v, o, do, lse, scale: float, causal):
    """Returns dQ, dK, dV (B, T, H, D) and D (B, H, T), float64."""
    Q, K, V, O, dO = (_bhtd(x) for x in (q, k, v, o, do))
    Ls = np.asarray(lse, dtype=np.float64)
    B, H = Q.shape[:2]
    G = _group(Q, K)
    dQ, dK, dV = np.empty_like(Q), np.zeros_like(K), np.zeros_like(V)
    Dv = np.empty(Ls.shape)
    for b in range(B):
        for h in range(H):
            dq, dk, dv, Dv[b, h] = bwd_head(
                Q[b, h], K[b, h // G], V[b, h // G], O[b, h], dO[b, h], Ls[b, h], scale, causal)
            dQ[b, h] = dq
            dK[b, h // G] += dk
            dV[b, h // G] += dv
    return _bthd(dQ), _bthd(dK), _bthd(dV), Dv


def attn_bwd_bwd_stats(q, k, v, o, do, ddq, ddk, ddv, lse, scale: float, causal,
                       return_stats: bool = False):
    """Returns dQ2, dK2, dV2, ddO (B, T, H, D) float64 [and D, dD, B (B, H, T)]."""
    Q, K, V, O, dO, ddQ, ddK, ddV = (_bhtd(x) for x in (q, k, v, o, do, ddq, ddk, ddv))
    Ls = np.asarray(lse, dtype=np.float64)
    B, H = Q.shape[:2]
    G = _group(Q, K)
    dQ2, dK2, dV2, ddO = np.empty_like(Q), np.zeros_like(K), np.zeros_like(V), np.empty_like(O)
    Dv, dDv, Bv = np.empty(Ls.shape), np.empty(Ls.shape), np.empty(Ls.shape)
    for b in range(B):
        for h in range(H):
            hk = h // G
            (dQ2[b, h], dk2, dv2, ddO[b, h],
             Dv[b, h], dDv[b, h], Bv[b, h]) = bwd_bwd_head(
                Q[b, h], K[b, hk], V[b, hk], O[b, h], dO[b, h],
                ddQ[b, h], ddK[b, hk], ddV[b, hk], Ls[b, h], scale, causal)
            dK2[b, hk] += dk2
            dV2[b, hk] += dv2
    outs = (_bthd(dQ2), _bthd(dK2), _bthd(dV2), _bthd(ddO))
    if return_stats:
        return outs + (Dv, dDv, Bv)
    return outs


def rel_err(actual, expected) -> float:
    """max|actual - expected| / max|expected| (0 if expected is all zero)."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    den = np.max(np.abs(e)) if e.size else 0.0
    num = np.max(np.abs(a - e)) if e.size else 0.0
    return float(num / den) if den > 0 else float(num)
