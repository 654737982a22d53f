"""Pins the CPU oracle before it is trusted as the checker (no GPU needed).

Each oracle function is checked against something other than a retyping of its own
formula: the reference's known-answer test, float64 brute force, a second independent
restatement in C, closed-form invariants, and the committed golden fixtures.
"""
import os

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import cref
from oracle import gemm as og
from oracle import int4 as oi

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ------------------------------------------------------------------------------- GEMM --
def test_kat_fragment_exact():
    # test_fragment_loading.py:237-256: C[i][k] = (i % 16) * 120 exactly.
    A, B, C = og.kat_fragment()
    assert torch.equal(og.gemm_ref(A, B), C)
    assert C[5, 7].item() == 5 * 120
    assert np.array_equal(cref.gemm(A.numpy(), B.numpy()), C.numpy())


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (1, 17, 9), (7, 5, 16), (16, 24, 33), (33, 9, 64)])
def test_gemm_ref_matches_f64_bruteforce(M, N, K):
    g = torch.Generator().manual_seed(42 + M + N + K)
    A = torch.randn(M, K, generator=g).half()
    B = torch.randn(K, N, generator=g).half()
    C = torch.randn(M, N, generator=g)
    ref64 = og.gemm_ref_f64(A.numpy(), B.numpy(), 2.0, 0.5, C.numpy())
    got = og.gemm_ref(A, B, 2.0, 0.5, C).double().numpy()
    assert np.allclose(got, ref64, rtol=1e-5, atol=1e-5 * max(1.0, np.abs(ref64).max()))
    got_c = cref.gemm(A.numpy(), B.numpy(), 2.0, 0.5, C.numpy())
    assert np.allclose(got_c, ref64, rtol=1e-5, atol=1e-5 * max(1.0, np.abs(ref64).max()))


def test_gemm_invariants():
    g = torch.Generator().manual_seed(7)
    A = torch.randn(48, 32, generator=g).half()
    B = torch.randn(32, 40, generator=g).half()
    # identity B returns A exactly
    assert torch.equal(og.gemm_ref(A, torch.eye(32).half()), A.float())
    # zero A gives zero
    assert torch.count_nonzero(og.gemm_ref(torch.zeros_like(A), B)) == 0
    # a column permutation of B permutes the columns of C
    perm = torch.randperm(40, generator=g)
    assert torch.equal(og.gemm_ref(A, B[:, perm]), og.gemm_ref(A, B)[:, perm])
    # linearity in alpha (power-of-two alpha is exact)
    assert torch.equal(og.gemm_ref(A, B, alpha=4.0), 4.0 * og.gemm_ref(A, B))


def test_gemm_beta_zero_never_reads_c():
    # wmma_gemm.hip:1914: C is read only if beta != 0 and C was given.
    A = torch.ones(4, 8).half()
    B = torch.ones(8, 4).half()
    C = torch.full((4, 4), float("nan"))
    out = og.gemm_ref(A, B, alpha=1.0, beta=0.0, C=C)
    assert torch.isfinite(out).all() and torch.equal(out, torch.full((4, 4), 8.0))
    out_c = cref.gemm(A.numpy(), B.numpy(), 1.0, 0.0, C.numpy())
    assert np.isfinite(out_c).all()
    # beta != 0 without C: beta ignored
    assert torch.equal(og.gemm_ref(A, B, alpha=2.0, beta=3.0, C=None), torch.full((4, 4), 16.0))


@pytest.mark.parametrize("K,split", [(4096, 1), (4096, 4), (4096, 16), (1000, 3), (64, 8), (4097, 32)])
def test_splitk_partition(K, split):
    # wmma_xor_swizzle.hpp:327: k_per_split = ceil(K / split); ranges cover [0, K) once.
    parts = og.splitk_partition(K, split)
    kps = -(-K // split)
    assert parts[0][0] == 0 and parts[-1][1] == K
    for (a0, a1), (b0, b1) in zip(parts, parts[1:]):
        assert a1 == b0
    assert all(b - a <= kps for a, b in parts)
    assert sum(b - a for a, b in parts) == K


def test_splitk_sum_equals_full_product():
    g = torch.Generator().manual_seed(3)
    A = torch.randint(-3, 4, (16, 256), generator=g).half()  # integer data: sums exact
    B = torch.randint(-3, 4, (256, 24), generator=g).half()
    full = og.gemm_ref(A, B)
    for split in (1, 2, 3, 4, 16):
        assert torch.equal(og.splitk_gemm_ref(A, B, split), full)
        assert np.array_equal(cref.gemm(A.numpy(), B.numpy(), split=split), full.numpy())


def test_max_rel_err_metric():
    ref = torch.tensor([[1.0, -4.0], [2.0, 0.0]])
    y = ref.clone()
    y[0, 1] = -3.9
    assert abs(og.max_rel_err(y, ref) - 0.1 / 4.0) < 1e-7
    assert og.max_rel_err(torch.zeros(2), torch.zeros(2)) == 0.0


# ------------------------------------------------------------------------------- INT4 --
def _rand_q(K, N, seed):
    return np.random.default_rng(seed).integers(0, 16, (K, N), dtype=np.uint8)


def test_pack_unpack_roundtrip_and_bit_positions():
    q = _rand_q(64, 40, 1)
    qw = oi.pack_gptq(q)
    assert qw.dtype == np.int32 and qw.shape == (8, 40)
    assert np.array_equal(oi.unpack_gptq(qw), q)
    # k = 8*row + j sits at bits 4j..4j+3 (GPTQ convention)
    assert ((qw[3, 5].astype(np.int64) & 0xFFFFFFFF) >> (4 * 6)) & 0xF == q[3 * 8 + 6, 5]
    assert np.array_equal(cref.pack_gptq(q), qw)


def test_single_nibble_positions():
    # one nonzero weight at every k offset: bit position moves as specified
    for k in range(8):
        q = np.zeros((8, 1), dtype=np.uint8)
        q[k, 0] = 0xA
        assert (int(oi.pack_gptq(q)[0, 0]) & 0xFFFFFFFF) == 0xA << (4 * k)


def test_zeros_pack_roundtrip():
    z = _rand_q(4, 64, 2)
    zp = oi.pack_zeros(z)
    assert zp.shape == (4, 8)
    assert np.array_equal(oi.unpack_zeros(zp), z)
    assert (int(zp[1, 2]) & 0xFFFFFFFF) >> 12 & 0xF == z[1, 2 * 8 + 3]


@pytest.mark.parametrize("K,N", [(64, 32), (128, 64), (256, 96), (512, 128)])
def test_prepack_bijection_and_c_restatement(K, N):
    q = _rand_q(K, N, K + N)
    qw = oi.pack_gptq(q)
    pk = oi.prepack(qw)
    assert pk.shape == (N // 16, K // 64, 32, 4) and pk.dtype == np.int32
    assert np.array_equal(oi.unprepack(pk), qw)
    assert np.array_equal(cref.prepack(qw).reshape(pk.shape), pk)  # independent C restatement
    # same multiset of nibbles
    nib = lambda a: np.sort(np.concatenate([(a.view(np.uint32) >> (4 * j)) & 0xF for j in range(8)], axis=None))
    assert np.array_equal(nib(pk), nib(qw))


def test_prepack_layout_spot_values():
    # slice s, block kc, entry l, word w <- GPTQ word kg = 8*kc + 4*(l//16) + w, column
    # 16*s + l%16, nibble p holds k-offset PERM[p].
    K, N = 128, 64
    q = _rand_q(K, N, 11)
    qw = oi.pack_gptq(q)
    pk = oi.prepack(qw).view(np.uint32).reshape(N // 16, K // 64, 32, 4)
    for (sl, kc, l, w) in [(0, 0, 0, 0), (3, 1, 31, 3), (1, 1, 17, 2), (2, 0, 9, 1)]:
        kg = 8 * kc + 4 * (l // 16) + w
        n = 16 * sl + l % 16
        word = int(pk[sl, kc, l, w])
        for p, koff in enumerate(oi.PERM):
            assert (word >> (4 * p)) & 0xF == q[8 * kg + koff, n]


def test_dequant_two_independent_routes():
    K, N, G = 256, 64, 64
    q = _rand_q(K, N, 5)
    z = _rand_q(K // G, N, 6)
    s = (np.random.default_rng(7).uniform(0.001, 0.02, (K // G, N))).astype(np.float16)
    a = oi.dequant(q, s, z, G)
    b = oi.dequant_f64_route(q, s, z, G)
    c = cref.dequant(q, s, z, G)
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))
    assert np.array_equal(a.view(np.uint16), c.view(np.uint16))


def test_dequant_special_cases():
    K, N, G = 64, 32, 32
    q = _rand_q(K, N, 8)
    s = np.full((K // G, N), 0.0123, dtype=np.float16)
    z_eq = q[::G].copy()  # z equal to the first row of each group
    w = oi.dequant(q, s, z_eq, G)
    assert np.all(w[::G] == 0)
    ones = np.ones((K // G, N), dtype=np.float16)
    w1 = oi.dequant(q, ones, np.zeros((K // G, N), dtype=np.uint8), G)
    assert np.array_equal(w1.astype(np.int32), q.astype(np.int32))


def test_w4a16_ref_against_c():
    A, q, s, z = oi.make_inputs(3, 128, 64, 64, seed=9)
    ref = oi.w4a16_ref(A, q, s, z, 64).numpy()
    W = cref.dequant(q, s, z, 64)
    got = cref.w4a16(A.numpy(), W)
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-5 * np.abs(ref).max())


def test_golden_int4_fixture():
    path = os.path.join(GOLDEN, "int4_k256_n64_g64.npz")
    d = np.load(path)
    q, s, z = d["q"], d["scales"], d["zeros_u8"]
    assert np.array_equal(oi.pack_gptq(q), d["qweight"])
    assert np.array_equal(oi.prepack(d["qweight"]).reshape(d["packed"].shape), d["packed"])
    assert np.array_equal(oi.pack_zeros(z), d["zeros_packed"])
    assert np.array_equal(oi.dequant(q, s, z, 64).view(np.uint16), d["w_fp16_bits"])
    A = torch.from_numpy(d["A"])
    assert np.allclose(oi.w4a16_ref(A, q, s, z, 64).numpy(), d["Y"], rtol=0, atol=0)


# -------------------------------------------------------------------------- attention --
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("Sq,Sk,D", [(8, 8, 16), (13, 13, 32), (5, 9, 16), (9, 5, 16)])
def test_sdpa_ref_matches_naive_f64(causal, Sq, Sk, D):
    Q, K, V = oatt.make_inputs(1, 2, Sq, D, seed=Sq * 7 + Sk, Sk=Sk)
    ref = oatt.attention_naive_f64(Q.numpy(), K.numpy(), V.numpy(), causal)
    got = oatt.sdpa_ref(Q, K, V, causal).double().numpy()
    assert np.allclose(got, ref, atol=2e-6)


def test_sdpa_invariants():
    Q, K, V = oatt.make_inputs(1, 1, 16, 16, seed=1)
    # identical V rows -> every output row equals that row
    Vc = V[:, :, :1, :].expand_as(V).contiguous()
    assert torch.allclose(oatt.sdpa_ref(Q, K, Vc), Vc.float(), atol=1e-6)
    # causal row 0 attends only key 0
    assert torch.allclose(oatt.sdpa_ref(Q, K, V, causal=True)[0, 0, 0], V[0, 0, 0].float(), atol=1e-6)
    # scale -> 0 gives the mean of V (uniform weights), prefix means when causal
    out = torch.nn.functional.scaled_dot_product_attention(Q.float(), K.float(), V.float(), scale=1e-30)
    assert torch.allclose(out[0, 0, 3], V.float()[0, 0].mean(0), atol=1e-5)
    outc = torch.nn.functional.scaled_dot_product_attention(Q.float(), K.float(), V.float(),
                                                            is_causal=True, scale=1e-30)
    assert torch.allclose(outc[0, 0, 3], V.float()[0, 0, :4].mean(0), atol=1e-5)
    # permuting keys together with values leaves the non-causal output unchanged
    perm = torch.randperm(16)
    assert torch.allclose(oatt.sdpa_ref(Q, K[:, :, perm], V[:, :, perm]), oatt.sdpa_ref(Q, K, V), atol=1e-6)
    # default scale is 1/sqrt(D)
    assert oatt.resolve_scale(128, -1.0) == pytest.approx(1 / np.sqrt(128))


# Grouped-query attention: key/value head j serves query heads j*g .. j*g+g-1.
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("H,Hkv", [(4, 2), (6, 1), (8, 4)])
def test_sdpa_ref_gqa_matches_torch_enable_gqa(causal, H, Hkv):
    Q, K, V = oatt.make_inputs(2, H, 11, 16, seed=H * 10 + Hkv, Sk=13, Hkv=Hkv)
    got = oatt.sdpa_ref(Q, K, V, causal)
    lib = torch.nn.functional.scaled_dot_product_attention(Q.float(), K.float(), V.float(),
                                                           is_causal=causal, enable_gqa=True)
    assert torch.allclose(got, lib, atol=1e-6)
    ref = oatt.attention_naive_f64(Q.numpy(), K.numpy(), V.numpy(), causal)
    assert np.allclose(got.double().numpy(), ref, atol=2e-6)


def test_gqa_head_mapping_closed_form():
    # V rows constant within each key/value head j (value c_j): every output of query head h
    # equals c_{h // g} (up to the rounding of the softmax weights' sum), whatever the
    # scores -- pins which head is read.
    H, Hkv, D = 6, 3, 16
    Q, K, _ = oatt.make_inputs(1, H, 7, D, seed=3, Hkv=Hkv)
    c = torch.arange(1, Hkv + 1, dtype=torch.float16).view(1, Hkv, 1, 1) * torch.ones(1, Hkv, 7, D).half()
    O = oatt.sdpa_ref(Q, K, c)
    for h in range(H):
        assert torch.allclose(O[0, h], torch.full_like(O[0, h], float(h // (H // Hkv) + 1)), atol=1e-6)


def test_slice_params_layout():
    # every element lands where the sliced layout puts it, and the layout is a bijection
    rng = np.random.default_rng(5)
    ng, N = 6, 64
    sc = rng.standard_normal((ng, N)).astype(np.float16)
    z = rng.integers(0, 16, (ng, N), dtype=np.uint8)
    s_sl, z_sl = oi.slice_params(sc, z)
    assert s_sl.shape == (N // 16, ng, 16) and z_sl.shape == (N // 16, ng, 2) and z_sl.dtype == np.int32
    zw = z_sl.view(np.uint32)
    for g in range(ng):
        for n in range(N):
            assert s_sl[n // 16, g, n % 16] == sc[g, n]
            assert (zw[n // 16, g, (n // 8) % 2] >> (4 * (n % 8))) & 0xF == z[g, n]
    assert sorted(s_sl.ravel().tolist()) == sorted(sc.ravel().tolist())
    # the packed-zeros words of a slice are the standard packed words, regrouped
    zp = oi.pack_zeros(z)
    assert np.array_equal(z_sl.reshape(N // 16, ng, 2).transpose(1, 0, 2).reshape(ng, N // 8), zp)


@pytest.mark.parametrize("K,N,G", [(512, 64, 128), (640, 32, 128), (4096, 32, 256), (1152, 96, 128),
                                   (2048, 64, 512)])
def test_fused_layout_closed_form(K, N, G):
    # Every weight nibble, scale and zero point lands at the byte the written layout gives
    # (an index formula independent of the oracle's construction), the buffer has exactly the
    # bytes of the separate tensors at G = 128, and unprepack_fused inverts it.
    rng = np.random.default_rng(K + N + G)
    q = rng.integers(0, 16, (K, N), dtype=np.uint8)
    sc = (rng.random((K // G, N)) * 0.02 + 0.001).astype(np.float16)
    z = rng.integers(0, 16, (K // G, N), dtype=np.uint8)
    qw = oi.pack_gptq(q)
    f = oi.prepack_fused(qw, sc, z, G)
    b = f.view(np.uint8).reshape(N // 16, -1)
    KP = K // 128
    hdr = -(-160 * (-(-KP // 4)) // 128) * 128  # 160 B per four K steps, up to 128 B lines
    assert b.shape[1] == hdr + 1024 * KP and hdr % 128 == 0
    if G == 128 and K % 4096 == 0:
        assert f.nbytes == K * N // 2 + (K // G) * N * 2 + (K // G) * N // 2
    for _ in range(300):
        k, n = int(rng.integers(K)), int(rng.integers(N))
        pp, sl, c = k // 128, n // 16, n % 16
        rec = (pp // 4) * 160
        # weight nibble: K step pp, block kc % 2, entry 16*h + c (h = (k % 64) // 32),
        # word (k % 32) // 8, nibble p with PERM[p] = k % 8
        kc = k // 64
        p_nib = oi.PERM.index(k % 8)
        off = hdr + pp * 1024 + (kc % 2) * 512 + (16 * ((k % 64) // 32) + c) * 16 + 4 * ((k % 32) // 8) + p_nib // 2
        assert (b[sl, off] >> (4 * (p_nib % 2))) & 0xF == q[k, n]
        g = k // G
        so = rec + 2 * (16 * (pp % 4) + c)
        assert int(b[sl, so]) | (int(b[sl, so + 1]) << 8) == int(sc[g, n].view(np.uint16))
        zo = rec + 128 + 8 * (pp % 4) + c // 2
        assert (b[sl, zo] >> (4 * (c % 2))) & 0xF == z[g, n]
    q2, s2, z2 = oi.unprepack_fused(f, K, G)
    assert np.array_equal(q2, qw) and np.array_equal(z2, z)
    assert np.array_equal(s2.view(np.uint16), sc.view(np.uint16))
    # the weights are the standard prepacked run of each slice, and the header padding is zero
    assert np.array_equal(b[:, hdr:], oi.prepack(qw).view(np.uint8).reshape(N // 16, KP * 1024))
    assert not b[:, 160 * (-(-KP // 4)):hdr].any()


def test_awq_pack_round_trip_and_order():
    rng = np.random.default_rng(11)
    q = rng.integers(0, 16, (32, 64), dtype=np.uint8)
    w = oi.pack_awq(q)
    assert w.shape == (32, 8) and w.dtype == np.int32
    assert np.array_equal(oi.unpack_awq(w), q)
    # a single nonzero column lands in the nibble AutoAWQ's order assigns it
    for col in range(8):
        one = np.zeros((1, 8), dtype=np.uint8)
        one[0, col] = 0xF
        nib = oi.AWQ_ORDER.index(col)
        assert int(oi.pack_awq(one).view(np.uint32)[0, 0]) == 0xF << (4 * nib)
    # the order is a permutation, and converting to the GPTQ layout keeps every value
    assert sorted(oi.AWQ_ORDER) == list(range(8))
    z = rng.integers(0, 16, (4, 64), dtype=np.uint8)
    qg, zp = oi.awq_to_gptq(oi.pack_awq(np.repeat(q, 1, axis=0)), oi.pack_awq(z))
    assert np.array_equal(oi.unpack_gptq(qg), q) and np.array_equal(oi.unpack_zeros(zp), z)


def test_sdpa_varlen_ref_equals_dense_for_equal_lengths():
    # equal-length packed sequences are the dense [B, H, S, D] problem, per sequence
    B, H, Hkv, S, D = 3, 4, 2, 9, 16
    Q, K, V = oatt.make_inputs(B, H, S, D, seed=21, Hkv=Hkv)
    cu = torch.arange(0, (B + 1) * S, S, dtype=torch.int32)
    pack = lambda X: X.transpose(1, 2).reshape(B * S, X.shape[1], D)
    for causal in (False, True):
        got = oatt.sdpa_varlen_ref(pack(Q), pack(K), pack(V), cu, cu, causal)
        want = pack(oatt.sdpa_ref(Q, K, V, causal))
        assert torch.allclose(got, want, atol=1e-6)
    # an empty sequence contributes nothing; a sequence without keys gives zeros
    cu_q = torch.tensor([0, 0, 5], dtype=torch.int32)
    cu_k = torch.tensor([0, 3, 3], dtype=torch.int32)
    q = torch.randn(5, 2, 8).half()
    kv = torch.randn(3, 2, 8).half()
    assert torch.count_nonzero(oatt.sdpa_varlen_ref(q, kv, kv, cu_q, cu_k)) == 0


# ------------------------------------------------------------------ attention training --
def _lse_naive_f64(Q, K, causal, scale=-1.0):
    Q = np.asarray(Q, dtype=np.float64)
    K = oatt.expand_kv(np.asarray(K, dtype=np.float64), Q.shape[1])
    S = np.einsum("...qd,...kd->...qk", Q, K) * oatt.resolve_scale(Q.shape[-1], scale)
    if causal:
        S = np.where(np.tril(np.ones(S.shape[-2:], dtype=bool)), S, -np.inf)
    m = S.max(axis=-1, keepdims=True)
    return (m + np.log(np.exp(S - m).sum(axis=-1, keepdims=True)))[..., 0]


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("Sq,Sk,H,Hkv", [(7, 7, 2, 2), (5, 9, 4, 2), (9, 5, 3, 1)])
def test_lse_ref_matches_naive_f64(causal, Sq, Sk, H, Hkv):
    Q, K, _ = oatt.make_inputs(2, H, Sq, 16, seed=Sq + 3 * Sk, Sk=Sk, Hkv=Hkv)
    got = oatt.lse_ref(Q, K, causal).double().numpy()
    assert np.allclose(got, _lse_naive_f64(Q.numpy(), K.numpy(), causal), atol=2e-6)


def _fd_grads(Q, K, V, dO, causal, eps=1e-6):
    """Central finite differences of f = sum(attention_naive_f64(Q, K, V) * dO), float64."""
    arrs = [np.asarray(X, dtype=np.float64).copy() for X in (Q, K, V)]
    dO = np.asarray(dO, dtype=np.float64)
    f = lambda: float((oatt.attention_naive_f64(*arrs, causal) * dO).sum())
    grads = []
    for X in arrs:
        g = np.zeros_like(X)
        for idx in np.ndindex(X.shape):
            x0 = X[idx]
            X[idx] = x0 + eps
            fp = f()
            X[idx] = x0 - eps
            fm = f()
            X[idx] = x0
            g[idx] = (fp - fm) / (2 * eps)
        grads.append(g)
    return grads


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("H,Hkv,Sq,Sk", [(2, 2, 5, 5), (4, 2, 4, 6), (2, 1, 6, 3)])
def test_sdpa_bwd_ref_matches_finite_differences(causal, H, Hkv, Sq, Sk):
    # Gradients pinned by float64 finite differences of the explicit forward -- a route that
    # shares nothing with autograd or with the dS = P (dP - Delta) closed form.
    D = 4
    Q, K, V = oatt.make_inputs(1, H, Sq, D, seed=H * 31 + Sq, Sk=Sk, Hkv=Hkv)
    dO = torch.randn(1, H, Sq, D, generator=torch.Generator().manual_seed(7)).half()
    want = _fd_grads(Q.numpy(), K.numpy(), V.numpy(), dO.numpy(), causal)
    got = oatt.sdpa_bwd_ref(Q, K, V, dO, causal)
    for g, w in zip(got, want):
        assert g.shape == w.shape
        assert np.allclose(g.double().numpy(), w, atol=2e-5 * max(1.0, np.abs(w).max()))


@pytest.mark.parametrize("causal", [False, True])
def test_sdpa_bwd_closed_forms(causal):
    # softmax rows sum to 1 -> the dV rows sum to the dO rows; softmax is invariant to a
    # per-row shift of the scores -> the dS rows sum to 0, so the dK rows sum to 0 and dQ
    # vanishes when every key is the same vector.
    B, H, Hkv, S, D = 2, 4, 2, 24, 16
    Q, K, V = oatt.make_inputs(B, H, S, D, seed=5, Hkv=Hkv)
    dO = torch.randn(B, H, S, D, generator=torch.Generator().manual_seed(8)).half()
    dQ, dK, dV = oatt.sdpa_bwd_ref(Q, K, V, dO, causal)
    dO_group = dO.float().view(B, Hkv, H // Hkv, S, D).sum(dim=(2, 3))
    assert torch.allclose(dV.sum(dim=2), dO_group, atol=1e-4)
    assert torch.allclose(dK.sum(dim=2), torch.zeros(B, Hkv, D), atol=1e-4)
    Kc = K[:, :, :1].expand_as(K).contiguous()
    dQc, _, _ = oatt.sdpa_bwd_ref(Q, Kc, V, dO, causal)
    assert dQc.abs().max() < 1e-5


def test_sdpa_varlen_bwd_ref_equals_dense():
    B, H, Hkv, S, D = 3, 4, 2, 9, 16
    Q, K, V = oatt.make_inputs(B, H, S, D, seed=22, Hkv=Hkv)
    dO = torch.randn(B, H, S, D, generator=torch.Generator().manual_seed(9)).half()
    cu = torch.arange(0, (B + 1) * S, S, dtype=torch.int32)
    pack = lambda X: X.transpose(1, 2).reshape(B * S, X.shape[1], D)
    for causal in (False, True):
        got = oatt.sdpa_varlen_bwd_ref(pack(Q), pack(K), pack(V), pack(dO), cu, cu, causal)
        want = oatt.sdpa_bwd_ref(Q, K, V, dO, causal)
        for g, w in zip(got, want):
            assert torch.allclose(g, pack(w), atol=1e-6)
        lse = oatt.lse_varlen_ref(pack(Q), pack(K), cu, cu, causal)
        assert torch.allclose(lse, oatt.lse_ref(Q, K, causal).permute(1, 0, 2).reshape(H, B * S))
    # a sequence without keys: +inf log-sum-exp and zero gradients
    cu_q = torch.tensor([0, 4, 6], dtype=torch.int32)
    cu_k = torch.tensor([0, 0, 3], dtype=torch.int32)
    q, dOq = torch.randn(6, 2, 8).half(), torch.randn(6, 2, 8).half()
    kv = torch.randn(3, 2, 8).half()
    lse = oatt.lse_varlen_ref(q, kv, cu_q, cu_k)
    assert torch.isinf(lse[:, :4]).all() and torch.isfinite(lse[:, 4:]).all()
    dq, _, _ = oatt.sdpa_varlen_bwd_ref(q, kv, kv, dOq, cu_q, cu_k)
    assert torch.count_nonzero(dq[:4]) == 0 and torch.count_nonzero(dq[4:]) > 0


# GPTQ checkpoint restatement: v1 zero offset and act-order g_idx, pinned by closed forms
# and by the native dequantisation (which it must reproduce when the layouts agree).
def test_gptq_v1_zero_offset_closed_forms():
    K, N, G = 256, 64, 64
    rng = np.random.default_rng(21)
    q = rng.integers(0, 16, (K, N), dtype=np.uint8)
    z = rng.integers(1, 16, (K // G, N), dtype=np.uint8)
    s = rng.uniform(0.001, 0.02, (K // G, N)).astype(np.float16)
    qz1 = oi.pack_gptq_v1_zeros(z)
    assert np.array_equal(oi.unpack_zeros(qz1), z - 1)                 # stored z - 1
    w1 = oi.gptq_dequant(oi.pack_gptq(q), qz1, s, None, v1=True)
    w2 = oi.gptq_dequant(oi.pack_gptq(q), oi.pack_zeros(z), s, None, v1=False)
    native = oi.dequant(q, s, z, G)
    assert np.array_equal(w1.view(np.uint16), native.view(np.uint16))
    assert np.array_equal(w2.view(np.uint16), native.view(np.uint16))
    # q == z (v1 storing z - 1) gives exactly zero; a plain layout g_idx equals none
    zq = np.repeat(z, G, axis=0)
    assert not np.any(oi.gptq_dequant(oi.pack_gptq(zq), qz1, s, None, v1=True))
    plain = np.arange(K) // G
    assert np.array_equal(oi.gptq_dequant(oi.pack_gptq(q), qz1, s, plain).view(np.uint16),
                          w1.view(np.uint16))


def test_gptq_act_order_rows_follow_g_idx():
    # Build an act-order checkpoint by scattering the rows of a plain one: row k of the
    # checkpoint is row rank[k] of the plain layout, where rank sorts the rows by group.
    K, N, G = 256, 32, 32
    rng = np.random.default_rng(22)
    q = rng.integers(0, 16, (K, N), dtype=np.uint8)
    z = rng.integers(1, 16, (K // G, N), dtype=np.uint8)
    s = rng.uniform(0.001, 0.02, (K // G, N)).astype(np.float16)
    g_idx = oi.act_order_g_idx(K, G, 5)
    assert np.array_equal(np.bincount(g_idx), np.full(K // G, G))
    perm = np.argsort(g_idx, kind="stable")           # sorted position -> checkpoint row
    rank = np.empty(K, dtype=np.int64)
    rank[perm] = np.arange(K)                          # checkpoint row -> sorted position
    assert np.array_equal(g_idx[perm], np.arange(K) // G)
    q_ckpt = q[rank]
    w = oi.gptq_dequant(oi.pack_gptq(q_ckpt), oi.pack_gptq_v1_zeros(z), s, g_idx)
    native = oi.dequant(q, s, z, G)
    assert np.array_equal(w[perm].view(np.uint16), native.view(np.uint16))
