"""Autodiff oracle: torch-CPU double VJP of materialised softmax attention.

TEST INFRASTRUCTURE ONLY (tests/, __graft_entry__.smoke(), bench.py's
cpu_baseline leg); never part of the product path.

This restates the reference's XLA oracle, tests/test_jax_fhog.py:14-34:
  reference_dpa       = jax.nn.dot_product_attention(..., implementation="xla")
  make_reference_dpa_bwd_bwd(q, k, v, do) = vjp of f(Q, K, V, dO) = vjp(attn)(dO),
  applied to the cotangents (ddQ, ddK, ddV) -> (dQ2, dK2, dV2, ddO).
JAX is absent here, so the same composition runs as torch autograd with
create_graph=True; it is a library routine independent of the closed-form
restatement in oracle/attention.py. In fp32 with one thread per host core it is
also the CPU baseline the GPU double backward is reported beside.
"""

from __future__ import annotations

import math

import torch


def attention(q, k, v, scale: float, causal):
    """Textbook attention on (B, T, H, D) tensors.

    causal: False/0 none, True/1 top-left (key j visible to query i iff
    j <= i), 2 bottom-right (j <= i + n_k - n_q). k and v may have fewer heads
    than q (a divisor): they are repeated per group of consecutive query heads
    (torch.repeat_interleave, the grouping of SDPA's enable_gqa), so autograd
    sums the key-side gradients over each group.
    """
    G = q.shape[2] // k.shape[2]
    if G > 1:
        k, v = k.repeat_interleave(G, dim=2), v.repeat_interleave(G, dim=2)
    s = torch.einsum("bqhd,bkhd->bhqk", q, k) * scale
    if causal:
        nq, nk = q.shape[1], k.shape[1]
        off = nk - nq if int(causal) == 2 else 0
        mask = torch.arange(nk)[None, :] <= torch.arange(nq)[:, None] + off
        s = s.masked_fill(~mask, float("-inf"))
    p = torch.softmax(s, dim=-1)
    return torch.einsum("bhqk,bkhd->bqhd", p, v)


def first_vjp(q, k, v, do, scale: float, causal: bool):
    q, k, v = (x.detach().requires_grad_(True) for x in (q, k, v))
    o = attention(q, k, v, scale, causal)
    return torch.autograd.grad(o, (q, k, v), do)


def double_vjp(q, k, v, do, ddq, ddk, ddv, scale: float, causal: bool):
    """(dQ2, dK2, dV2, ddO) = vjp of (Q,K,V,dO) -> vjp(attn)(dO) at (ddQ,ddK,ddV)."""
    q, k, v, do = (x.detach().requires_grad_(True) for x in (q, k, v, do))
    o = attention(q, k, v, scale, causal)
    dq, dk, dv = torch.autograd.grad(o, (q, k, v), do, create_graph=True)
    return torch.autograd.grad((dq, dk, dv), (q, k, v, do), (ddq, ddk, ddv))


def double_vjp_chunked(q, k, v, do, ddq, ddk, ddv, scale: float, causal: bool, heads_per_chunk: int = 1):
    """double_vjp over (B, T, H, D) tensors, a few heads at a time to bound memory."""
    B, _, H, _ = q.shape
    outs = [torch.empty_like(q), torch.empty_like(k), torch.empty_like(v), torch.empty_like(do)]
    for b in range(B):
        for h0 in range(0, H, heads_per_chunk):
            sl = (slice(b, b + 1), slice(None), slice(h0, h0 + heads_per_chunk))
            res = double_vjp(q[sl], k[sl], v[sl], do[sl], ddq[sl], ddk[sl], ddv[sl], scale, causal)
            for dst, r in zip(outs, res):
                dst[sl] = r
    return tuple(outs)


def unmasked_pairs(n_q: int, n_k: int, causal) -> int:
    """Number of (query, key) pairs that survive the mask, per (batch, head):
    query i sees min(n_k, max(0, i + 1 + off)) keys, off = 0 top-left (causal
    1 or True), n_k - n_q bottom-right (causal 2)."""
    if not causal:
        return n_q * n_k
    off = n_k - n_q if int(causal) == 2 else 0
    # sum over i of clamp(i + 1 + off, 0, n_k): a ramp, then a plateau at n_k
    lo = max(0, -off)                     # first query that sees a key
    ramp_end = min(n_q, max(lo, n_k - off - 1))  # queries [lo, ramp_end) see i + 1 + off < n_k keys
    a, b = lo + 1 + off, ramp_end + off   # first and last ramp counts
    ramp = (a + b) * (ramp_end - lo) // 2 if ramp_end > lo else 0
    return ramp + (n_q - ramp_end) * n_k


def bwdbwd_algorithmic_flops(batch, heads, n_q, n_k, head_dim, causal) -> float:
    """24 * head_dim flops per unmasked pair: the 12 distinct (N_Q x N_K x d)
    products of the double backward, recomputation not counted."""
    return 24.0 * head_dim * batch * heads * unmasked_pairs(n_q, n_k, causal)


def default_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)
