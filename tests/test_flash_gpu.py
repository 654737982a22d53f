"""GPU parity of flash-attention forward against fp32 CPU SDPA (max rel err <= 1e-3)."""
import math

import numpy as np

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


# The same configuration checked on every one of its 128 (batch, head) slices against the
# fp32 CPU reference, eight heads per CPU call; the error is the global max-relative metric.
@pytest.mark.parametrize("causal", [False, True])
def test_flash_baseline_config_all_heads(wo, causal):
    B, H, S, D = 4, 32, 4096, 128
    report("flash_all_heads", B=B, H=H, S=S, D=D, causal=causal)
    Q, K, V = oatt.make_inputs(B, H, S, D, seed=42 + 4)
    O = wo.flash_attention(Q.cuda(), K.cuda(), V.cuda(), causal=causal,
                           scale=1.0 / math.sqrt(D)).cpu().float()
    worst, peak = 0.0, 0.0
    for b in range(B):
        for h in range(0, H, 8):
            ref = oatt.sdpa_ref(Q[b:b + 1, h:h + 8], K[b:b + 1, h:h + 8], V[b:b + 1, h:h + 8], causal)
            worst = max(worst, (O[b:b + 1, h:h + 8] - ref).abs().max().item())
            peak = max(peak, ref.abs().max().item())
    assert worst / peak <= TOL, f"max rel err {worst / peak:.3e}"


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("B,H,Sq,Sk,D", [(2, 8, 512, 512, 64), (1, 4, 77, 77, 128), (2, 2, 200, 200, 64),
                                         (1, 3, 100, 300, 128), (1, 2, 300, 100, 64), (1, 1, 1, 1, 128),
                                         (1, 2, 129, 129, 128)])
def test_flash_shapes(wo, causal, B, H, Sq, Sk, D):
    report("flash_shape", B=B, H=H, Sq=Sq, Sk=Sk, D=D, causal=causal)
    Q, K, V = oatt.make_inputs(B, H, Sq, D, seed=Sq + Sk + D, Sk=Sk)
    O = wo.flash_attention(Q.cuda(), K.cuda(), V.cuda(), causal=causal)
    _check(O, oatt.sdpa_ref(Q, K, V, causal))


# Head dims other than the kernels' 64, 128 and 256: multiples of 8 run on the smallest
# kernel that holds them with the missing d columns loaded as zeros and not stored; other
# sizes are zero-padded to a multiple of 8 by the torch layer.  Default scale 1/sqrt(D) of the
# caller's D throughout.  Ragged Sq != Sk, both masks, grouped-query heads.
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("D", [8, 16, 24, 32, 40, 48, 56, 72, 80, 96, 104, 112, 120, 1, 33, 100, 127,
                               136, 160, 192, 200, 248, 256, 129, 250])
def test_flash_head_dims(wo, causal, D):
    B, H, Hkv, Sq, Sk = 2, 4, 2, 200, 333
    report("flash_head_dim", B=B, H=H, Hkv=Hkv, Sq=Sq, Sk=Sk, D=D, causal=causal)
    Q, K, V = oatt.make_inputs(B, H, Sq, D, seed=500 + D, Sk=Sk, Hkv=Hkv)
    O, lse = wo.flash_attention_forward(Q.cuda(), K.cuda(), V.cuda(), causal)
    _check(O, oatt.sdpa_ref(Q, K, V, causal))
    ref_lse = oatt.lse_ref(Q, K, causal)
    assert torch.allclose(lse.cpu(), ref_lse, atol=1e-4, rtol=1e-5), (lse.cpu() - ref_lse).abs().max()
    assert torch.equal(O, wo.flash_attention(Q.cuda(), K.cuda(), V.cuda(), causal=causal))


# The padded head dims leave the rows past D untouched: a head-dim-80 problem computes the
# same bits as the same problem zero-padded to 128 by the caller, cut back to 80 columns.
def test_flash_head_dim_equals_padded(wo):
    B, H, S, D = 2, 3, 300, 80
    Q, K, V = oatt.make_inputs(B, H, S, D, seed=77)
    pad = lambda X: torch.nn.functional.pad(X, (0, 128 - D)).cuda()
    for causal in (False, True):
        O = wo.flash_attention(Q.cuda(), K.cuda(), V.cuda(), causal=causal)
        Op = wo.flash_attention(pad(Q), pad(K), pad(V), causal=causal, scale=1.0 / math.sqrt(D))
        assert torch.equal(O, Op[..., :D])
        assert torch.count_nonzero(Op[..., D:]) == 0


# D = 256 (4 waves, 2-deep ring) at a longer sequence: many key tiles through the ring,
# ragged ends, grouped-query heads, both masks.
@pytest.mark.parametrize("causal", [False, True])
def test_flash_head_dim_256(wo, causal):
    B, H, Hkv, Sq, Sk, D = 2, 8, 2, 1000, 1300, 256
    report("flash_d256", B=B, H=H, Hkv=Hkv, Sq=Sq, Sk=Sk, D=D, causal=causal)
    Q, K, V = oatt.make_inputs(B, H, Sq, D, seed=256, Sk=Sk, Hkv=Hkv)
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


# Variable-length packed batches ([total, heads, D] with cu_seqlens): ragged lengths
# (including 1 and lengths that are not multiples of the 64-key tile or 256-query block),
# an empty sequence, different query and key lengths, grouped-query heads, both head sizes.
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("H,Hkv,D", [(8, 8, 128), (8, 2, 64), (6, 3, 128), (4, 2, 80), (6, 6, 40),
                                     (4, 1, 100)])
def test_flash_varlen(wo, causal, H, Hkv, D):
    lens_q = [300, 1, 0, 1000, 64, 257]
    lens_k = [300, 1, 5, 1000, 77, 700]
    report("flash_varlen", H=H, Hkv=Hkv, D=D, causal=causal)
    cu_q = torch.tensor([0] + list(np.cumsum(lens_q)), dtype=torch.int32)
    cu_k = torch.tensor([0] + list(np.cumsum(lens_k)), dtype=torch.int32)
    g = torch.Generator().manual_seed(H * 10 + D)
    q = torch.randn(int(cu_q[-1]), H, D, generator=g).half()
    k = torch.randn(int(cu_k[-1]), Hkv, D, generator=g).half()
    v = torch.randn(int(cu_k[-1]), Hkv, D, generator=g).half()
    O = wo.flash_attention_varlen(q.cuda(), k.cuda(), v.cuda(), cu_q.cuda(), cu_k.cuda(),
                                  max(lens_q), max(lens_k), causal=causal)
    ref = oatt.sdpa_varlen_ref(q, k, v, cu_q, cu_k, causal)
    assert O.dtype == torch.float16 and O.shape == q.shape
    assert torch.isfinite(O).all()
    err = og.max_rel_err(O.float().cpu(), ref)
    assert err <= TOL, err


def test_flash_varlen_equals_dense(wo):
    # equal lengths: the packed problem is the dense one, computed to the same bits
    B, H, S, D = 3, 4, 333, 128
    Q, K, V = oatt.make_inputs(B, H, S, D, seed=12)
    pack = lambda X: X.transpose(1, 2).reshape(B * S, H, D).contiguous().cuda()
    cu = torch.arange(0, (B + 1) * S, S, dtype=torch.int32).cuda()
    for causal in (False, True):
        dense = wo.flash_attention(Q.cuda(), K.cuda(), V.cuda(), causal=causal)
        packed = wo.flash_attention_varlen(pack(Q), pack(K), pack(V), cu, cu, S, S, causal=causal)
        assert torch.equal(packed, dense.transpose(1, 2).reshape(B * S, H, D))


def test_flash_errors(wo):
    for D in (264, 512):
        x = torch.zeros(1, 1, 8, D, dtype=torch.half, device="cuda")
        with pytest.raises(RuntimeError, match="head_dim must be between 1 and 256"):
            wo.flash_attention(x, x, x)
    y = torch.zeros(1, 1, 8, 64, dtype=torch.float32, device="cuda")
    with pytest.raises(RuntimeError, match="float16"):
        wo.flash_attention(y, y, y)
    q = torch.zeros(1, 6, 8, 64, dtype=torch.half, device="cuda")
    kv = torch.zeros(1, 4, 8, 64, dtype=torch.half, device="cuda")
    with pytest.raises(RuntimeError, match="K/V heads must divide Q heads"):
        wo.flash_attention(q, kv, kv)
    p = torch.zeros(8, 2, 64, dtype=torch.half, device="cuda")
    cu = torch.tensor([0, 8], dtype=torch.int64, device="cuda")
    with pytest.raises(RuntimeError, match="cu_seqlens must be int32"):
        wo.flash_attention_varlen(p, p, p, cu, cu, 8, 8)


# More work items (batch*head x 256-query blocks) than CUs, so several waves of workgroups
# share each CU: ragged lengths, Sq != Sk, grouped-query heads, and query blocks with fewer
# key tiles than the 4-deep ring (Sk = 100: two key tiles).
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("B,H,Hkv,Sq,Sk,D", [(2, 64, 64, 1000, 1000, 128), (4, 64, 16, 700, 300, 64),
                                             (1, 300, 300, 256, 100, 128), (8, 40, 8, 513, 513, 64)])
def test_flash_many_items(wo, causal, B, H, Hkv, Sq, Sk, D):
    report("flash_many_items", B=B, H=H, Hkv=Hkv, Sq=Sq, Sk=Sk, D=D, causal=causal)
    Q, K, V = oatt.make_inputs(B, H, Sq, D, seed=B * H + Sq + Sk, Sk=Sk, Hkv=Hkv)
    O, lse = wo.flash_attention_forward(Q.cuda(), K.cuda(), V.cuda(), causal)
    assert torch.isfinite(O).all()
    g = H // Hkv
    for b, h in [(0, 0), (B - 1, H - 1), (B // 2, H // 2), (0, H - 1)]:
        j = h // g
        ref = oatt.sdpa_ref(Q[b:b + 1, h:h + 1], K[b:b + 1, j:j + 1], V[b:b + 1, j:j + 1], causal)
        _check(O[b:b + 1, h:h + 1], ref)
        lref = oatt.lse_ref(Q[b:b + 1, h:h + 1], K[b:b + 1, j:j + 1], causal)
        assert torch.allclose(lse[b:b + 1, h:h + 1].cpu(), lref, atol=1e-4, rtol=1e-5)
    # the inference entry point computes the same bits
    assert torch.equal(O, wo.flash_attention(Q.cuda(), K.cuda(), V.cuda(), causal))


# Decoding shapes (few queries, many keys): the forward splits the key range over more
# workgroups and merges the chunks (wmma_flash_attn_fwd_ws; the torch layer always passes
# the workspace).  Checked against the CPU oracle (O and lse) and against the one-pass
# forward of the same inputs through the C-ABI (no workspace); causal shapes whose later
# chunks hold no live key (top-left alignment), GQA, ragged Sk, head dims 64-256.
@pytest.mark.parametrize("B,H,Hkv,Sq,Sk,D,causal", [
    (1, 32, 32, 1, 4096, 128, False), (1, 32, 8, 1, 8192, 128, False), (2, 8, 2, 4, 3000, 64, False),
    (1, 16, 16, 16, 4096, 256, False), (1, 8, 8, 3, 5003, 72, True), (1, 4, 4, 200, 4096, 128, True),
    (1, 32, 32, 1, 600, 128, False), (3, 4, 4, 2, 2048, 128, True)])
def test_flash_decode_split(wo, B, H, Hkv, Sq, Sk, D, causal):
    import ctypes
    lib = ctypes.CDLL(wo.LIBRARY_PATH)
    vp, i32, f32, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
    lib.wmma_flash_attn_fwd_workspace_size.restype = sz
    lib.wmma_flash_attn_fwd_workspace_size.argtypes = [i32] * 7
    lib.wmma_flash_attn_fwd_lse.argtypes = [vp] * 5 + [i32] * 6 + [f32, i32, vp]
    need = lib.wmma_flash_attn_fwd_workspace_size(B, H, Hkv, Sq, Sk, D, 1 if causal else 0)
    report("flash_decode_split", B=B, H=H, Hkv=Hkv, Sq=Sq, Sk=Sk, D=D, causal=causal, ws=need)
    assert need > 0, "the shape should take the split path"
    Q, K, V = oatt.make_inputs(B, H, Sq, D, seed=Sq * 7 + Sk, Sk=Sk, Hkv=Hkv)
    Qd, Kd, Vd = Q.cuda(), K.cuda(), V.cuda()
    O, lse = wo.flash_attention_forward(Qd, Kd, Vd, causal=causal)
    ref = oatt.sdpa_ref(Q, K, V, causal)
    _check(O.cpu(), ref)
    lref = oatt.lse_ref(Q, K, causal)
    fin = torch.isfinite(lref)
    assert torch.equal(torch.isfinite(lse.cpu()), fin)
    assert (lse.cpu()[fin] - lref[fin]).abs().max().item() <= 1e-3
    assert torch.equal(wo.flash_attention(Qd, Kd, Vd, causal=causal), O)
    # the one-pass forward of the same inputs (C-ABI without a workspace)
    O1 = torch.empty_like(Qd)
    lse1 = torch.empty(B, H, Sq, device="cuda")
    rc = lib.wmma_flash_attn_fwd_lse(Qd.data_ptr(), Kd.data_ptr(), Vd.data_ptr(), O1.data_ptr(),
                                     lse1.data_ptr(), B, H, Hkv, Sq, Sk, D, 1.0 / math.sqrt(D),
                                     1 if causal else 0, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    _check(O1.cpu(), ref)
    assert og.max_rel_err(O.float(), O1.float()) <= 1e-3


# Grouped-query heads without a causal mask run as one sequence per K/V head (each K/V tile
# read once per group): the same query rows compute the same arithmetic, so the result is
# bit-identical to multi-head attention on K/V expanded to every query head (both through
# the one-pass C-ABI forward, no workspace), lse included.
@pytest.mark.parametrize("B,H,Hkv,Sq,Sk,D", [(2, 8, 2, 300, 300, 128), (1, 32, 8, 1, 4096, 128),
                                             (2, 6, 3, 77, 100, 64), (1, 4, 1, 513, 640, 256)])
def test_flash_gqa_packed_equals_expanded(wo, B, H, Hkv, Sq, Sk, D):
    import ctypes
    report("flash_gqa_packed", B=B, H=H, Hkv=Hkv, Sq=Sq, Sk=Sk, D=D)
    lib = ctypes.CDLL(wo.LIBRARY_PATH)
    vp, i32, f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
    lib.wmma_flash_attn_fwd_lse.argtypes = [vp] * 5 + [i32] * 6 + [f32, i32, vp]
    Q, K, V = oatt.make_inputs(B, H, Sq, D, seed=B + H + Sq, Sk=Sk, Hkv=Hkv)
    Qd, Kd, Vd = Q.cuda(), K.cuda(), V.cuda()
    Kx, Vx = oatt.expand_kv(K, H).contiguous().cuda(), oatt.expand_kv(V, H).contiguous().cuda()
    st = torch.cuda.current_stream().cuda_stream
    outs = []
    for kk, vv, hkv in ((Kd, Vd, Hkv), (Kx, Vx, H)):
        O = torch.empty_like(Qd)
        lse = torch.empty(B, H, Sq, device="cuda")
        assert lib.wmma_flash_attn_fwd_lse(Qd.data_ptr(), kk.data_ptr(), vv.data_ptr(), O.data_ptr(),
                                           lse.data_ptr(), B, H, hkv, Sq, Sk, D, 1.0 / math.sqrt(D), 0, st) == 0
        outs.append((O, lse))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    _check(outs[0][0].cpu(), oatt.sdpa_ref(Q, K, V, False))
