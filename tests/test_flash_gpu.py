"""GPU parity of flash-attention forward against fp32 CPU SDPA (max rel err <= 1e-3)."""
import math

import pytest
import torch

from oracle import attention as oatt
from oracle import gemm as og
from tests.conftest import report

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _check(O, ref):
    assert O.dtype == torch.float16 and tuple(O.shape) == tuple(ref.shape)
    assert torch.isfinite(O).all()
    err = og.max_rel_err(O.float(), ref)
    assert err <= TOL, f"max rel err {err:.3e}"
    return err


# [4, 32, 4096, 128], scale 1/sqrt(128), causal and non-causal.  The CPU
# reference is evaluated on a sample of (batch, head) pairs at the full sequence length.
@pytest.mark.parametrize("causal", [False, True])
def test_flash_baseline_config(wo, causal):
    B, H, S, D = 4, 32, 4096, 128
    report("flash", B=B, H=H, S=S, D=D, causal=causal)
    Q, K, V = oatt.make_inputs(B, H, S, D, seed=42 + 4)
    O = wo.flash_attention(Q.cuda(), K.cuda(), V.cuda(), causal=causal, scale=1.0 / math.sqrt(D))
    assert torch.isfinite(O).all()
    assert O.abs().max().item() <= V.abs().max().item() * (1 + 1e-3)
    for b, h in [(0, 0), (1, 17), (3, 31)]:
        ref = oatt.sdpa_ref(Q[b:b + 1, h:h + 1], K[b:b + 1, h:h + 1], V[b:b + 1, h:h + 1], causal)
        _check(O[b:b + 1, h:h + 1], ref)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("B,H,Sq,Sk,D", [(2, 8, 512, 512, 64), (1, 4, 77, 77, 128), (2, 2, 200, 200, 64),
                                         (1, 3, 100, 300, 128), (1, 2, 300, 100, 64), (1, 1, 1, 1, 128),
                                         (1, 2, 129, 129, 128)])
def test_flash_shapes(wo, causal, B, H, Sq, Sk, D):
    report("flash_shape", B=B, H=H, Sq=Sq, Sk=Sk, D=D, causal=causal)
    Q, K, V = oatt.make_inputs(B, H, Sq, D, seed=Sq + Sk + D, Sk=Sk)
    O = wo.flash_attention(Q.cuda(), K.cuda(), V.cuda(), causal=causal)
    _check(O, oatt.sdpa_ref(Q, K, V, causal))


def test_flash_custom_scale(wo):
    Q, K, V = oatt.make_inputs(2, 4, 256, 64, seed=3)
    O = wo.flash_attention(Q.cuda(), K.cuda(), V.cuda(), False, 0.1)
    _check(O, oatt.sdpa_ref(Q, K, V, False, 0.1))


def test_flash_invariants(wo):
    Q, K, V = oatt.make_inputs(1, 2, 256, 128, seed=5)
    Vc = V[:, :, :1, :].expand_as(V).contiguous()
    O = wo.flash_attention(Q.cuda(), K.cuda(), Vc.cuda())
    assert torch.allclose(O.float().cpu(), Vc.float(), atol=2e-3)
    Oc = wo.flash_attention(Q.cuda(), K.cuda(), V.cuda(), causal=True)
    assert torch.allclose(Oc[0, :, 0].float().cpu(), V[0, :, 0].float(), atol=1e-3)


# Scores that climb by ~46 (in log2 units) every 64-key tile, and isolated spikes late in
# the sequence: the running max must move mid-sequence (rescale of O and the row sum, tile
# recomputed) -- the path ordinary N(0,1) inputs only take on the first tile.
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("pattern", ["ramp", "spikes"])
def test_flash_running_max_moves(wo, causal, pattern):
    B, H, S, D = 1, 2, 1024, 128
    g = torch.Generator().manual_seed(11)
    Q = (torch.ones(B, H, S, D) + 0.1 * torch.randn(B, H, S, D, generator=g))
    if pattern == "ramp":
        t = 0.05 * torch.arange(S, dtype=torch.float32)          # score ~ 0.57 * key index
        K = torch.ones(B, H, S, D) * t[None, None, :, None]
    else:
        K = 0.5 * torch.randn(B, H, S, D, generator=g)
        K[:, :, [300, 301, 700, 1000]] += 6.0                      # +68 in the score
    V = torch.randn(B, H, S, D, generator=g)
    Q, K, V = Q.half(), K.half(), V.half()
    report("flash_max_moves", pattern=pattern, causal=causal)
    O = wo.flash_attention(Q.cuda(), K.cuda(), V.cuda(), causal=causal)
    _check(O, oatt.sdpa_ref(Q, K, V, causal))


# Grouped-query / multi-query attention: K and V carry Hkv heads, query head h reads
# key/value head h // (H / Hkv) (torch SDPA's enable_gqa mapping).
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("B,H,Hkv,Sq,Sk,D", [(2, 8, 2, 300, 300, 128), (1, 8, 1, 257, 257, 64),
                                             (2, 4, 4, 128, 128, 64), (1, 6, 3, 100, 333, 128),
                                             (1, 32, 8, 1024, 1024, 128)])
def test_flash_gqa(wo, causal, B, H, Hkv, Sq, Sk, D):
    report("flash_gqa", B=B, H=H, Hkv=Hkv, Sq=Sq, Sk=Sk, D=D, causal=causal)
    Q, K, V = oatt.make_inputs(B, H, Sq, D, seed=H * 100 + Hkv + Sq, Sk=Sk, Hkv=Hkv)
    O = wo.flash_attention(Q.cuda(), K.cuda(), V.cuda(), causal=causal)
    _check(O, oatt.sdpa_ref(Q, K, V, causal))


def test_flash_gqa_head_mapping(wo):
    # V constant within each key/value head j (value j + 1): query head h must output
    # h // g + 1 everywhere (to within the rounding of the softmax weights), whatever the
    # scores.
    H, Hkv, D = 8, 2, 64
    Q, K, _ = oatt.make_inputs(2, H, 200, D, seed=9, Hkv=Hkv)
    V = (torch.arange(1, Hkv + 1, dtype=torch.float16).view(1, Hkv, 1, 1)
         * torch.ones(2, Hkv, 200, D)).half()
    O = wo.flash_attention(Q.cuda(), K.cuda(), V.cuda(), causal=True).cpu()
    for h in range(H):
        want = float(h // (H // Hkv) + 1)
        assert torch.allclose(O[:, h].float(), torch.full((2, 200, D), want), atol=2e-3 * want), h


def test_flash_errors(wo):
    x = torch.zeros(1, 1, 8, 96, dtype=torch.half, device="cuda")
    with pytest.raises(RuntimeError, match="head_dim"):
        wo.flash_attention(x, x, x)
    y = torch.zeros(1, 1, 8, 64, dtype=torch.float32, device="cuda")
    with pytest.raises(RuntimeError, match="float16"):
        wo.flash_attention(y, y, y)
    q = torch.zeros(1, 6, 8, 64, dtype=torch.half, device="cuda")
    kv = torch.zeros(1, 4, 8, 64, dtype=torch.half, device="cuda")
    with pytest.raises(RuntimeError, match="K/V heads must divide Q heads"):
        wo.flash_attention(q, kv, kv)
