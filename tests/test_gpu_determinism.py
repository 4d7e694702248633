"""Determinism and exact sharding of the double backward.

Both kernels are atomic-free: every output element is accumulated by one wave
in a fixed order, and every (batch, key/value head) pair is computed by its own
workgroups from its own inputs. Hence, bit for bit:

- repeated calls on the same inputs give the same outputs and row statistics;
- the batch can be split into shards (each shard a separate call) and the
  shards' outputs equal the corresponding slices of the unsplit call;
- heads can be split the same way, in whole key/value-head groups for grouped
  queries (query head h reads key/value head h / (H / H_kv));
- the order in which a grid takes its blocks (plain or in chunks of
  (batch, head) pairs, chosen from the grid's size) does not change any output.

The last two are the sharding over (B, H) that needs no exchange between
devices (the reference's multi-device test shards the batch,
tests/test_jax_fhog.py:194-237).
"""

from __future__ import annotations

import math

import pytest
import torch

from helpers import make_inputs

pytestmark = pytest.mark.gpu

CASES = [
    # name, B, N, H, H_kv, dtype, causal (0 none, 1 top-left)
    ("bf16_causal", 4, 384, 4, 4, torch.bfloat16, 1),
    ("f16_noncausal_ragged", 3, 200, 2, 2, torch.float16, 0),
    ("bf16_gqa_causal", 2, 320, 8, 2, torch.bfloat16, 1),
]


def _announce(*what):
    print("[case]", *what, flush=True)


def _run(x, causal, scale):
    from flash_hog import _hip

    o, lse = _hip.attention_fwd(x["q"], x["k"], x["v"], causal, scale)
    dq2, dk2, dv2, ddo, stats = _hip.attention_bwdbwd(x["q"], x["k"], x["v"], o, x["do"], x["ddq"], x["ddk"],
                                                      x["ddv"], lse, causal, scale, return_stats=True)
    return (o, lse, dq2, dk2, dv2, ddo) + tuple(stats)


def _slice(x, b=slice(None), h=None, hk=None):
    """Contiguous copies of a batch / head slice of the inputs."""
    out = {}
    for name, t in x.items():
        sel = h if name in ("q", "do", "ddq") else hk
        u = t[b]
        if sel is not None:
            u = u[:, :, sel]
        out[name] = u.contiguous()
    return out


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_repeat_and_shard_bit_exact(case):
    name, B, N, H, Hkv, dtype, causal = case
    _announce("determinism", name, B, N, H, Hkv)
    dev = torch.device("cuda:0")
    D = 64
    scale = 1.0 / math.sqrt(D)
    x = make_inputs(B, N, N, H, D, dtype, seed=7, device=dev, kv_heads=Hkv)
    ref = _run(x, causal, scale)
    again = _run(x, causal, scale)
    for a, r in zip(again, ref):
        assert torch.equal(a, r), "repeated call differs"

    # batch shards: one sample per call
    for b in range(B):
        part = _run(_slice(x, b=slice(b, b + 1)), causal, scale)
        for a, r in zip(part, ref):
            # o, lse, dq2..ddo are batch-major; the row statistics are (B, H, T)
            assert torch.equal(a, r[b:b + 1]), f"batch shard {b} differs"

    # head shards: whole key/value-head groups per call
    grp = H // Hkv
    for hk in range(Hkv):
        hs = slice(hk * grp, (hk + 1) * grp)
        part = _run(_slice(x, h=hs, hk=slice(hk, hk + 1)), causal, scale)
        o, lse, dq2, dk2, dv2, ddo, *stats = part
        ro, rlse, rdq2, rdk2, rdv2, rddo, *rstats = ref
        assert torch.equal(o, ro[:, :, hs]) and torch.equal(lse, rlse[:, hs]), f"forward head shard {hk} differs"
        assert torch.equal(dq2, rdq2[:, :, hs]) and torch.equal(ddo, rddo[:, :, hs]), f"head shard {hk}: dQ2/ddO"
        assert torch.equal(dk2, rdk2[:, :, hk:hk + 1]) and torch.equal(dv2, rdv2[:, :, hk:hk + 1]), \
            f"head shard {hk}: dK2/dV2"
        for s, rs in zip(stats, rstats):
            assert torch.equal(s, rs[:, hs]), f"head shard {hk}: row statistics"


# Grids of more than 8 rounds of resident workgroups (256 CUs, two workgroups
# per CU) take the (batch, head) pairs in chunks, the last chunk short here;
# a one-sample call takes the plain order. Each workgroup's arithmetic does not
# depend on its place in the grid, so every sample of the large call equals its
# own one-sample call bit for bit: forward, first backward and double backward.
LARGE = [
    # name, B, N, H, H_kv, dtype, causal
    ("bf16_causal_b130", 130, 512, 16, 16, torch.bfloat16, 1),
    ("f16_gqa_noncausal_ragged_b140", 140, 300, 8, 2, torch.float16, 0),
]


def _run_all(x, causal, scale):
    from flash_hog import _hip

    out = _run(x, causal, scale)
    o, lse = out[0], out[1]
    return out + tuple(_hip.attention_bwd(x["q"], x["k"], x["v"], o, x["do"], lse, causal, scale))


@pytest.mark.parametrize("case", LARGE, ids=[c[0] for c in LARGE])
def test_chunked_grid_equals_per_sample(case):
    name, B, N, H, Hkv, dtype, causal = case
    _announce("grid order", name, B, N, H, Hkv)
    dev = torch.device("cuda:0")
    D = 64
    scale = 1.0 / math.sqrt(D)
    x = make_inputs(B, N, N, H, D, dtype, seed=11, device=dev, kv_heads=Hkv)
    ref = _run_all(x, causal, scale)
    for b in range(B):
        part = _run_all(_slice(x, b=slice(b, b + 1)), causal, scale)
        for i, (a, r) in enumerate(zip(part, ref)):
            assert torch.equal(a, r[b:b + 1]), f"sample {b}, output {i}"
