"""The torch entry points under HIP graph capture: every replay equals the eager result.

Each case runs the call eagerly, captures the same call into a torch.cuda.CUDAGraph (its
output, and any split-K or flash workspace, come from the graph's private pool), then
replays the graph three times with unrelated eager work and a synchronisation between the
replays, and checks every replay bit-for-bit against the eager output.  The cases cover
each kernel family the planners pick at these shapes and every workspace-using path: the
tiled GEMM with and without a K split, the skinny GEMM and its reduction, a two-part plan,
the alpha/beta epilogue, W4A16 decode (standard and fused layouts), skinny and tiled with a
K split, flash forward (including the split-key-range decode path with its merge kernel)
and the flash backward (dQ and dK/dV kernels; a grouped-query split).  Every path is
deterministic, so bit equality is the bar; the eager result itself is checked against the
oracle elsewhere (test_gemm_gpu, test_w4a16_gpu, test_flash_gpu, test_flash_bwd_gpu).
"""
import math

import pytest
import torch

from oracle import attention as oatt
from oracle import int4 as oi
from tests.conftest import report

pytestmark = pytest.mark.gpu


def _replays_match(fn, replays=3):
    """Eager result, then a captured graph of the same call replayed `replays` times."""
    eager = fn()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up on a side stream, as torch's capture expects
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    noise = torch.randn(1 << 20, device="cuda")
    for r in range(replays):
        graph.replay()
        torch.cuda.synchronize()
        outs = out if isinstance(out, (tuple, list)) else (out,)
        refs = eager if isinstance(eager, (tuple, list)) else (eager,)
        for o, e in zip(outs, refs):
            assert torch.equal(o, e), f"replay {r} differs from the eager result"
        noise.mul_(1.0001).add_(0.5)  # eager work between replays
        torch.cuda.synchronize()


# (M, N, K): tiled 64x64 split 4, tiled 256x256, skinny split 8, skinny two-block split,
# tiled 128x64 split 4, a two-part plan (bulk 256x256 + edge GEMM)
GEMM_SHAPES = [(64, 4096, 4096), (1024, 1024, 2048), (1, 4096, 4096), (32, 14336, 4096),
               (128, 4096, 4096), (4100, 1024, 512)]


@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
def test_graph_matmul(wo, M, N, K):
    report("graph_matmul", M=M, N=N, K=K, plan=wo.gemm_plan(M, N, K))
    g = torch.Generator().manual_seed(M + N + K)
    A = torch.randn(M, K, generator=g).half().cuda()
    B = (torch.randn(K, N, generator=g) * 0.05).half().cuda()
    _replays_match(lambda: wo.matmul(A, B))


@pytest.mark.parametrize("M,N,K", [(128, 4096, 4096), (512, 512, 512)])
def test_graph_gemm_epilogue(wo, M, N, K):
    report("graph_gemm", M=M, N=N, K=K)
    g = torch.Generator().manual_seed(M + 2 * N + K)
    A = torch.randn(M, K, generator=g).half().cuda()
    B = (torch.randn(K, N, generator=g) * 0.05).half().cuda()
    C = torch.randn(M, N, generator=g).cuda()
    _replays_match(lambda: wo.gemm(A, B, 2.0, 0.5, C))


# W4A16 at configs[3] K: decode (M = 1, 2), skinny (16), tiled with a K split (256 at
# N = 4096), without (300), the rows kernel (128 at N = 4096, 300 at N = 1024)
@pytest.mark.parametrize("M,N", [(1, 4096), (2, 1024), (16, 4096), (256, 4096), (300, 4096), (128, 4096),
                                 (300, 1024)])
def test_graph_matmul_int4(wo, M, N):
    K, G = 4096, 128
    report("graph_w4a16", M=M, N=N, K=K, plan=wo.w4a16_plan(M, N, K, G))
    A, q, s, z = oi.make_inputs(M, K, N, G, seed=M + N)
    qd = torch.from_numpy(oi.pack_gptq(q)).cuda()
    sd, zd = torch.from_numpy(s).cuda(), torch.from_numpy(oi.pack_zeros(z)).cuda()
    pk, Ad = wo.prepack_int4(qd), A.cuda()
    _replays_match(lambda: wo.matmul_int4(Ad, pk, sd, zd, G))
    if M <= 4:
        f = wo.prepack_int4_fused(qd, sd, zd, G)
        _replays_match(lambda: wo.matmul_int4_fused(Ad, f, G))


# forward: [1,8,1024,128] causal and not; a decoding shape (Sq = 1 against 4096 keys, the
# split-key-range path and its merge kernel); grouped-query heads
@pytest.mark.parametrize("B,H,Hkv,Sq,Sk,causal", [(1, 8, 8, 1024, 1024, False),
                                                    (1, 8, 8, 1024, 1024, True),
                                                    (1, 32, 32, 1, 4096, False),
                                                    (2, 16, 4, 512, 512, False)])
def test_graph_flash_forward(wo, B, H, Hkv, Sq, Sk, causal):
    report("graph_flash_fwd", B=B, H=H, Hkv=Hkv, Sq=Sq, Sk=Sk, causal=causal)
    g = torch.Generator().manual_seed(B + H + Sq + Sk)
    Q = torch.randn(B, H, Sq, 128, generator=g).half().cuda()
    K = torch.randn(B, Hkv, Sk, 128, generator=g).half().cuda()
    V = torch.randn(B, Hkv, Sk, 128, generator=g).half().cuda()
    _replays_match(lambda: wo.flash_attention(Q, K, V, causal))


@pytest.mark.parametrize("B,H,Hkv,S,D,causal", [(1, 8, 8, 512, 128, False),
                                                 (1, 8, 8, 512, 64, True),
                                                 (1, 16, 2, 1024, 128, True)])
def test_graph_flash_backward(wo, B, H, Hkv, S, D, causal):
    report("graph_flash_bwd", B=B, H=H, Hkv=Hkv, S=S, D=D, causal=causal)
    Q, K, V = oatt.make_inputs(B, H, S, D, seed=B + H + S, Hkv=Hkv)
    Qd, Kd, Vd = Q.cuda(), K.cuda(), V.cuda()
    dO = torch.randn(B, H, S, D, generator=torch.Generator().manual_seed(7)).half().cuda()
    sc = 1.0 / math.sqrt(D)
    O, lse = wo.flash_attention_forward(Qd, Kd, Vd, causal, sc)
    _replays_match(lambda: wo.flash_attention_backward(dO, Qd, Kd, Vd, O, lse, causal, sc))
