"""fp32 closed-form attention forward, first and double backward on the GPU,
one head at a time.

A checker for the full-size configurations, where the numpy fp64 oracle would
take minutes: the same equations as oracle/attention.py (attn_fwd, attn_bwd,
bwd_bwd_head; flash_hog/_jax_refs/jax_impl.py:112-191, 301-336),
materialising (N_Q, N_K) fp32 matrices for one (batch, head) at a time. Each
function is pinned against the fp64 oracle in
tests/test_gpu_parity.py::test_gpu_reference_matches_oracle.
"""

from __future__ import annotations

import torch


def _mask(n_q, n_k, device):
    return torch.arange(n_k, device=device)[None, :] <= torch.arange(n_q, device=device)[:, None]


def bwdbwd_head(q, k, v, o, do, ddq, ddk, ddv, lse, scale, causal):
    mm = torch.mm
    s = mm(q, k.t().contiguous()) * scale
    if causal:
        s = s.masked_fill(~_mask(q.shape[0], k.shape[0], q.device), float("-inf"))
    p = torch.exp(s - lse[:, None])
    dp = mm(do, v.t().contiguous())
    dds = scale * (mm(ddq, k.t().contiguous()) + mm(q, ddk.t().contiguous()))
    d = (o * do).sum(-1)
    dd = (dds * p).sum(-1)
    dp2 = mm(do, ddv.t().contiguous()) - dp * dd[:, None] - dds * d[:, None] + dp * dds
    b = (dp2 * p).sum(-1)
    ds = scale * p * (dp - d[:, None])
    ds2 = scale * p * (dp2 - b[:, None])
    ddp = p * (dds - dd[:, None])
    dq2 = mm(ds, ddk) + mm(ds2, k)
    dk2 = mm(ds.t().contiguous(), ddq) + mm(ds2.t().contiguous(), q)
    dv2 = mm(ddp.t().contiguous(), do)
    ddo = mm(p, ddv) + mm(ddp, v)
    return dq2, dk2, dv2, ddo


def fwd_head(q, k, v, scale, causal):
    s = torch.mm(q, k.t().contiguous()) * scale
    if causal:
        s = s.masked_fill(~_mask(q.shape[0], k.shape[0], q.device), float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    return torch.mm(torch.exp(s - lse[:, None]), v), lse


def bwd_head(q, k, v, o, do, lse, scale, causal):
    """First backward (flash_hog/_jax_refs/jax_impl.py:142-191): dQ, dK, dV and D = rowsum(O dO)."""
    mm = torch.mm
    s = mm(q, k.t().contiguous()) * scale
    if causal:
        s = s.masked_fill(~_mask(q.shape[0], k.shape[0], q.device), float("-inf"))
    p = torch.exp(s - lse[:, None])
    dp = mm(do, v.t().contiguous())
    d = (o * do).sum(-1)
    ds = scale * p * (dp - d[:, None])
    return mm(ds, k), mm(ds.t().contiguous(), q), mm(p.t().contiguous(), do), d


def bwd(q, k, v, o, do, lse, scale, causal, heads=None):
    """(B, T, N, H) inputs -> fp32 dQ, dK, dV (B, T, N, H) and D (B, N, T) on the
    listed (batch, head) pairs (default: all); other entries are zero."""
    f = lambda x: x.float()
    q, k, v, o, do, lse = map(f, (q, k, v, o, do, lse))
    B, T, H, _ = q.shape
    outs = [torch.zeros_like(q), torch.zeros_like(k), torch.zeros_like(v), torch.zeros((B, H, T), device=q.device)]
    for b, h in heads if heads is not None else [(b, h) for b in range(B) for h in range(H)]:
        args = [x[b, :, h, :].contiguous() for x in (q, k, v, o, do)]
        dq, dk, dv, d = bwd_head(*args, lse[b, h].contiguous(), scale, causal)
        outs[0][b, :, h, :], outs[1][b, :, h, :], outs[2][b, :, h, :], outs[3][b, h] = dq, dk, dv, d
    return tuple(outs)


def bwdbwd(q, k, v, o, do, ddq, ddk, ddv, lse, scale, causal):
    """(B, T, N, H) inputs of any float dtype -> fp32 dQ2, dK2, dV2, ddO."""
    f = lambda x: x.float()
    q, k, v, o, do, ddq, ddk, ddv, lse = map(f, (q, k, v, o, do, ddq, ddk, ddv, lse))
    outs = [torch.empty_like(q), torch.empty_like(k), torch.empty_like(v), torch.empty_like(do)]
    B, _, H, _ = q.shape
    for b in range(B):
        for h in range(H):
            args = [x[b, :, h, :].contiguous() for x in (q, k, v, o, do, ddq, ddk, ddv)]
            res = bwdbwd_head(*args, lse[b, h].contiguous(), scale, causal)
            for dst, r in zip(outs, res):
                dst[b, :, h, :] = r
    return tuple(outs)


def fwd(q, k, v, scale, causal, heads=None):
    """(B, T, N, H) inputs -> fp32 O (B, T, N, H) and natural-log L (B, N, T) on
    the listed (batch, head) pairs (default: all); other entries are zero."""
    q, k, v = q.float(), k.float(), v.float()
    B, T, H, D = q.shape
    o = torch.zeros((B, T, H, v.shape[-1]), device=q.device)
    lse = torch.zeros((B, H, T), device=q.device)
    for b, h in heads if heads is not None else [(b, h) for b in range(B) for h in range(H)]:
        o[b, :, h, :], lse[b, h] = fwd_head(q[b, :, h, :].contiguous(), k[b, :, h, :].contiguous(),
                                            v[b, :, h, :].contiguous(), scale, causal)
    return o, lse


# ------------------------------------------------- row-chunked (long sequences)
#
# The same equations with the (N_Q, N_K) matrices formed `rows` query rows at a
# time, for sequences whose full matrices would not fit: every row statistic
# (L, D, dD, B) and every query-side output (O, dQ2, ddO) depends on its own
# rows only, and the key-side outputs (dK2, dV2) are sums over query rows, so
# they accumulate chunk by chunk. A causal chunk of rows [r0, r1) needs keys
# [0, r1) only (top-left mask, N_Q == N_K). Checked against the unchunked
# functions in tests/test_gpu_parity.py::test_gpu_reference_chunked.

def _chunk_keys(r1, n_k, causal):
    return min(r1, n_k) if causal else n_k


def fwd_head_chunked(q, k, v, scale, causal, rows=1024):
    o = torch.empty((q.shape[0], v.shape[1]), device=q.device)
    lse = torch.empty(q.shape[0], device=q.device)
    for r0 in range(0, q.shape[0], rows):
        r1 = min(r0 + rows, q.shape[0])
        nk = _chunk_keys(r1, k.shape[0], causal)
        s = torch.mm(q[r0:r1], k[:nk].t().contiguous()) * scale
        if causal:
            s = s.masked_fill(torch.arange(nk, device=q.device)[None, :] > torch.arange(r0, r1, device=q.device)[:, None],
                              float("-inf"))
        lse[r0:r1] = torch.logsumexp(s, dim=-1)
        o[r0:r1] = torch.mm(torch.exp(s - lse[r0:r1, None]), v[:nk])
        del s
    return o, lse


def bwdbwd_head_chunked(q, k, v, o, do, ddq, ddk, ddv, lse, scale, causal, rows=1024):
    mm = torch.mm
    dq2, ddo = torch.empty_like(q), torch.empty_like(do)
    dk2, dv2 = torch.zeros_like(k), torch.zeros_like(v)
    for r0 in range(0, q.shape[0], rows):
        r1 = min(r0 + rows, q.shape[0])
        nk = _chunk_keys(r1, k.shape[0], causal)
        kc, vc, ddkc, ddvc = k[:nk], v[:nk], ddk[:nk], ddv[:nk]
        qr, dor, ddqr = q[r0:r1], do[r0:r1], ddq[r0:r1]
        s = mm(qr, kc.t().contiguous()) * scale
        if causal:
            s = s.masked_fill(torch.arange(nk, device=q.device)[None, :] > torch.arange(r0, r1, device=q.device)[:, None],
                              float("-inf"))
        p = torch.exp(s - lse[r0:r1, None])
        del s
        dp = mm(dor, vc.t().contiguous())
        dds = scale * (mm(ddqr, kc.t().contiguous()) + mm(qr, ddkc.t().contiguous()))
        d = (o[r0:r1] * dor).sum(-1)
        dd = (dds * p).sum(-1)
        dp2 = mm(dor, ddvc.t().contiguous()) - dp * dd[:, None] - dds * d[:, None] + dp * dds
        b = (dp2 * p).sum(-1)
        ds = scale * p * (dp - d[:, None])
        ds2 = scale * p * (dp2 - b[:, None])
        ddp = p * (dds - dd[:, None])
        del dp, dp2, dds
        dq2[r0:r1] = mm(ds, ddkc) + mm(ds2, kc)
        ddo[r0:r1] = mm(p, ddvc) + mm(ddp, vc)
        dk2[:nk] += mm(ds.t().contiguous(), ddqr) + mm(ds2.t().contiguous(), qr)
        dv2[:nk] += mm(ddp.t().contiguous(), dor)
        del p, ds, ds2, ddp
    return dq2, dk2, dv2, ddo
