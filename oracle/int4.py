"""INT4 / W4A16 oracle (CPU, numpy).  Test infrastructure only -- see oracle/__init__.py.

The reference has no INT4 code (no name, layout or test to follow).  The semantics here
are the task's W4A16 definition and this library's written layout specification
(include/wmma_ops_amd.h):

  GPTQ qweight  int32 [K/8, N]; q[k][n] = (qweight[k//8][n] >> 4*(k%8)) & 0xF
  packed zeros  int32 [K/G, N/8]; z[g][n] = (zeros[g][n//8] >> 4*(n%8)) & 0xF
  prepacked     int32 [N/16][K/64][32][4]; slice s, block kc, entry l, word w holds the
                GPTQ word of k-group kg = 8*kc + 4*(l//16) + w for column 16*s + l%16,
                with its nibbles reordered: nibble p holds k-offset PERM[p]
  dequant       W[k][n] = fp16((q - z) * s), q - z exact, one rounding to fp16
  W4A16         Y = A.float() @ W.float()   (fp32 accumulate)
"""
from __future__ import annotations

import numpy as np
import torch

PERM = (0, 2, 4, 6, 1, 3, 5, 7)  # nibble position -> k offset inside a prepacked word


def pack_gptq(q: np.ndarray) -> np.ndarray:
    """uint8 q [K, N] (values 0..15) -> int32 qweight [K/8, N]."""
    q = np.asarray(q, dtype=np.uint32)
    K, N = q.shape
    assert K % 8 == 0
    q = q.reshape(K // 8, 8, N)
    out = np.zeros((K // 8, N), dtype=np.uint32)
    for j in range(8):
        out |= (q[:, j, :] & 0xF) << np.uint32(4 * j)
    return out.view(np.int32)


def unpack_gptq(qweight: np.ndarray) -> np.ndarray:
    """int32 qweight [K/8, N] -> uint8 q [K, N]."""
    w = np.asarray(qweight).view(np.uint32)
    kg, N = w.shape
    out = np.empty((kg, 8, N), dtype=np.uint8)
    for j in range(8):
        out[:, j, :] = (w >> np.uint32(4 * j)) & 0xF
    return out.reshape(kg * 8, N)


def pack_zeros(z: np.ndarray) -> np.ndarray:
    """uint8 z [K/G, N] -> int32 [K/G, N/8], nibble n%8 of word n//8."""
    z = np.asarray(z, dtype=np.uint32)
    ng, N = z.shape
    assert N % 8 == 0
    z = z.reshape(ng, N // 8, 8)
    out = np.zeros((ng, N // 8), dtype=np.uint32)
    for j in range(8):
        out |= (z[:, :, j] & 0xF) << np.uint32(4 * j)
    return out.view(np.int32)


# AutoAWQ (GEMM checkpoint format; AutoAWQ 0.2.x, not installed here) packs eight columns
# per int32 along N: column 8c + AWQ_ORDER[i] in nibble i, for qweight [K, N/8] and qzeros
# [K/G, N/8] alike (its packing code's AWQ_ORDER / AWQ_REVERSE_ORDER).  Restated from that
# published order; no AutoAWQ fixture exists here, so the adapter's parity is unpinned by
# an AutoAWQ run and pinned only by this restatement and round trips.
AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)


def pack_awq(q: np.ndarray) -> np.ndarray:
    """uint8 [R, N] (0..15) -> int32 [R, N/8] in AutoAWQ's nibble order."""
    q = np.asarray(q, dtype=np.uint32)
    R, N = q.shape
    assert N % 8 == 0
    q = q.reshape(R, N // 8, 8)
    out = np.zeros((R, N // 8), dtype=np.uint32)
    for i, col in enumerate(AWQ_ORDER):
        out |= (q[:, :, col] & 0xF) << np.uint32(4 * i)
    return out.view(np.int32)


def unpack_awq(w: np.ndarray) -> np.ndarray:
    """Inverse of pack_awq: int32 [R, N/8] -> uint8 [R, N]."""
    w = np.asarray(w).view(np.uint32)
    R, C = w.shape
    out = np.zeros((R, C, 8), dtype=np.uint8)
    for i, col in enumerate(AWQ_ORDER):
        out[:, :, col] = (w >> np.uint32(4 * i)) & 0xF
    return out.reshape(R, C * 8)


def awq_to_gptq(qweight_awq: np.ndarray, qzeros_awq: np.ndarray):
    """AutoAWQ qweight/qzeros -> (GPTQ-layout qweight [K/8, N], packed zeros [K/G, N/8])."""
    return pack_gptq(unpack_awq(qweight_awq)), pack_zeros(unpack_awq(qzeros_awq))


# GPTQ checkpoints.  AutoGPTQ's "gptq" format (v1; AutoGPTQ 0.7.x, not installed here) keeps
# qweight [K/8, N] (q[k][n] in nibble k%8 of word [k//8][n]) and scales [K/G, N] in this
# library's layout, but its packing code subtracts 1 from each zero point before packing it
# into qzeros [K/G, N/8] (nibble n%8 of word [g][n//8]) and its dequantisation adds the 1
# back: W[k][n] = (q[k][n] - (stored + 1)) * s.  GPTQModel's "gptq_v2" stores z itself.
# Act-order (desc_act) checkpoints carry g_idx [K], the group of each row.  Restated from
# that published packing and dequantisation; no GPTQ fixture exists here, so the adapter's
# parity with a GPTQ run is unpinned and rests on these restatements and closed forms.
def pack_gptq_v1_zeros(z: np.ndarray) -> np.ndarray:
    """uint8 zero points z [K/G, N] (1..16) -> v1 qzeros int32 [K/G, N/8] holding z - 1."""
    z = np.asarray(z, dtype=np.int32)
    assert z.min() >= 1 and z.max() <= 16, "v1 stores z - 1 in four bits"
    return pack_zeros((z - 1).astype(np.uint8))


def gptq_dequant(qweight: np.ndarray, qzeros: np.ndarray, scales: np.ndarray, g_idx,
                 v1: bool = True) -> np.ndarray:
    """GPTQ dequantisation W [K, N] fp16: fp16((q[k][n] - z[g_idx[k]][n]) * s[g_idx[k]][n]),
    z = stored nibble + 1 (v1) or stored nibble (v2); g_idx None means k // G."""
    q = unpack_gptq(qweight).astype(np.int32)
    K, N = q.shape
    z = unpack_zeros(qzeros).astype(np.int32) + (1 if v1 else 0)
    G = K // z.shape[0]
    g = np.arange(K) // G if g_idx is None else np.asarray(g_idx, dtype=np.int64)
    return (q - z[g, :]).astype(np.float16) * np.asarray(scales, dtype=np.float16)[g, :]


def gptq_w4a16_ref(A: torch.Tensor, qweight, qzeros, scales, g_idx, v1: bool = True) -> torch.Tensor:
    """Y = A.float() @ gptq_dequant(...).float(), fp32 on the CPU."""
    W = torch.from_numpy(gptq_dequant(qweight, qzeros, scales, g_idx, v1).astype(np.float32))
    return torch.matmul(A.detach().cpu().float(), W)


def act_order_g_idx(K: int, G: int, seed: int) -> np.ndarray:
    """A desc_act g_idx: rows visited in a random order, the i-th visited row in group i // G
    (how GPTQ assigns groups when it quantises columns by decreasing Hessian diagonal)."""
    order = np.random.default_rng(seed).permutation(K)
    g_idx = np.empty(K, dtype=np.int32)
    g_idx[order] = np.arange(K) // G
    return g_idx


def slice_params(s: np.ndarray, z: np.ndarray):
    """Slice-major group parameters (this library's WMMA_ZEROS_SLICED layout):
    scales fp16 [K/G, N] -> [N/16, K/G, 16]; uint8 zeros [K/G, N] -> int32 [N/16, K/G, 2]
    where word w of (slice i, group g) packs z[g][16 i + 8 w + j] into nibble j."""
    s = np.asarray(s)
    z = np.asarray(z, dtype=np.uint8)
    ng, N = s.shape
    assert N % 16 == 0 and z.shape == (ng, N)
    s_sl = np.ascontiguousarray(s.reshape(ng, N // 16, 16).transpose(1, 0, 2))
    z_sl = pack_zeros(z.reshape(ng, N // 16, 16).transpose(1, 0, 2).reshape(N // 16 * ng, 16))
    return s_sl, np.ascontiguousarray(z_sl.reshape(N // 16, ng, 2))


def unpack_zeros(zp: np.ndarray) -> np.ndarray:
    w = np.asarray(zp).view(np.uint32)
    ng, n8 = w.shape
    out = np.empty((ng, n8, 8), dtype=np.uint8)
    for j in range(8):
        out[:, :, j] = (w >> np.uint32(4 * j)) & 0xF
    return out.reshape(ng, n8 * 8)


def _permute_word_nibbles(w: np.ndarray, inverse: bool = False) -> np.ndarray:
    w = np.asarray(w, dtype=np.uint32)
    out = np.zeros_like(w)
    for p, koff in enumerate(PERM):
        if not inverse:  # nibble p of the result holds k-offset PERM[p] of the source
            out |= ((w >> np.uint32(4 * koff)) & 0xF) << np.uint32(4 * p)
        else:
            out |= ((w >> np.uint32(4 * p)) & 0xF) << np.uint32(4 * koff)
    return out


def prepack(qweight: np.ndarray) -> np.ndarray:
    """GPTQ qweight [K/8, N] -> prepacked int32 [N/16, K/64, 32, 4]."""
    w = np.asarray(qweight).view(np.uint32)
    kg, N = w.shape
    K = kg * 8
    assert K % 64 == 0 and N % 32 == 0
    KC, NS = K // 64, N // 16
    # w[kg, n] with kg = 8*kc + 4*h + word, n = 16*s + c  ->  out[s, kc, 16*h + c, word]
    t = w.reshape(KC, 2, 4, NS, 16)            # [kc, h, word, s, c]
    t = t.transpose(3, 0, 1, 4, 2)             # [s, kc, h, c, word]
    t = _permute_word_nibbles(t)
    return np.ascontiguousarray(t).reshape(NS, KC, 32, 4).view(np.int32)


def unprepack(packed: np.ndarray) -> np.ndarray:
    """Inverse of prepack: int32 [N/16, K/64, 32, 4] -> GPTQ qweight [K/8, N]."""
    p = np.asarray(packed).view(np.uint32)
    NS, KC = p.shape[0], p.shape[1]
    assert p.shape == (NS, KC, 32, 4)
    kg, N = KC * 8, NS * 16
    t = p.reshape(NS, KC, 2, 16, 4)            # [s, kc, h, c, word]
    t = _permute_word_nibbles(t, inverse=True)
    t = t.transpose(1, 2, 4, 0, 3)             # [kc, h, word, s, c]
    return np.ascontiguousarray(t).reshape(kg, N).view(np.int32)


# Fused decode layout (this library's WMMA_W4_FUSED, include/wmma_ops_amd.h): per 16-column
# slice, a header of one 160-byte parameter block per four 128-deep K steps (128 bytes of
# scales [4][16] fp16, 32 bytes of zero nibbles [4][16], even column low), zero-padded to a
# multiple of 128 bytes, then the slice's prepacked weights (1 KB per K step).
FUSED_BLOCK = 160


def fused_hdr_bytes(K: int) -> int:
    return (FUSED_BLOCK * ((K // 128 + 3) // 4) + 127) // 128 * 128


def fused_slice_bytes(K: int) -> int:
    return fused_hdr_bytes(K) + (K // 128) * 1024


def prepack_fused(qweight: np.ndarray, scales: np.ndarray, zeros_u8: np.ndarray, G: int) -> np.ndarray:
    """GPTQ qweight [K/8, N] + scales fp16 [K/G, N] + uint8 zeros [K/G, N] -> int32
    [N/16, fused_slice_bytes(K)/4].  K step pp (128 values of K) carries the parameters of
    group pp*128 // G; the weights are the slice's standard prepacked run."""
    pk = prepack(qweight)
    NS, KC = pk.shape[:2]
    K = KC * 64
    assert K % 128 == 0 and G % 128 == 0 and K % G == 0
    KP, H = K // 128, fused_hdr_bytes(K)
    out = np.zeros((NS, fused_slice_bytes(K)), dtype=np.uint8)
    out[:, H:] = pk.view(np.uint8).reshape(NS, KP * 1024)
    s16 = np.ascontiguousarray(np.asarray(scales, dtype=np.float16)).view(np.uint16)
    z = np.asarray(zeros_u8, dtype=np.uint8)
    for pp in range(KP):
        r, u = divmod(pp, 4)
        base, g = r * FUSED_BLOCK, pp * 128 // G
        out[:, base + 32 * u: base + 32 * (u + 1)] = (
            np.ascontiguousarray(s16[g].reshape(NS, 16)).view(np.uint8).reshape(NS, 32))
        zz = z[g].reshape(NS, 8, 2)
        out[:, base + 128 + 8 * u: base + 128 + 8 * (u + 1)] = (zz[:, :, 0] & 0xF) | ((zz[:, :, 1] & 0xF) << 4)
    return out.view(np.int32)


def unprepack_fused(fused: np.ndarray, K: int, G: int):
    """Inverse of prepack_fused -> (qweight [K/8, N] int32, scales fp16 [K/G, N], uint8
    zeros [K/G, N]); each group's parameters are read from its first K step."""
    b = np.ascontiguousarray(fused).view(np.uint8)
    NS = b.shape[0]
    KC, H = K // 64, fused_hdr_bytes(K)
    assert b.shape[1] == fused_slice_bytes(K)
    qweight = unprepack(np.ascontiguousarray(b[:, H:]).view(np.int32).reshape(NS, KC, 32, 4))
    KG = K // G
    s = np.empty((KG, NS * 16), dtype=np.uint16)
    z = np.empty((KG, NS * 16), dtype=np.uint8)
    for g in range(KG):
        r, u = divmod(g * G // 128, 4)
        base = r * FUSED_BLOCK
        s[g] = np.ascontiguousarray(b[:, base + 32 * u: base + 32 * (u + 1)]).view(np.uint16).reshape(-1)
        zb = b[:, base + 128 + 8 * u: base + 128 + 8 * (u + 1)]
        z[g] = np.stack([zb & 0xF, zb >> 4], axis=-1).reshape(-1)
    return qweight, s.view(np.float16), z


def dequant(q: np.ndarray, scales: np.ndarray, zeros_u8: np.ndarray, G: int) -> np.ndarray:
    """fp16((q - z) * s): the difference is exact in fp16 and numpy's float16 multiply
    rounds the exact product once."""
    q = np.asarray(q, dtype=np.int32)
    K, N = q.shape
    g = np.arange(K) // G
    z = np.asarray(zeros_u8, dtype=np.int32)[g, :]
    s = np.asarray(scales, dtype=np.float16)[g, :]
    return (q - z).astype(np.float16) * s


def dequant_f64_route(q: np.ndarray, scales: np.ndarray, zeros_u8: np.ndarray, G: int) -> np.ndarray:
    """The same value by an independent route: exact float64 product, one rounding."""
    q = np.asarray(q, dtype=np.float64)
    K, _ = q.shape
    g = np.arange(K) // G
    z = np.asarray(zeros_u8, dtype=np.float64)[g, :]
    s = np.asarray(scales, dtype=np.float16).astype(np.float64)[g, :]
    return ((q - z) * s).astype(np.float16)


def w4a16_ref(A: torch.Tensor, q: np.ndarray, scales: np.ndarray, zeros_u8: np.ndarray,
              G: int) -> torch.Tensor:
    """Y = A.float() @ W.float(), W = dequant(...), fp32 on the CPU."""
    W = torch.from_numpy(dequant(q, scales, zeros_u8, G).astype(np.float32))
    return torch.matmul(A.detach().cpu().float(), W)


def make_inputs(M: int, K: int, N: int, G: int, seed: int):
    """Seeded W4A16 inputs as the task describes them: A ~ N(0,1) fp16; q ~ U{0..15};
    s ~ U(0.001, 0.02) fp16; z ~ U{0..15}."""
    g = torch.Generator().manual_seed(seed)
    A = torch.randn(M, K, generator=g).half()
    q = torch.randint(0, 16, (K, N), generator=g, dtype=torch.int32).numpy().astype(np.uint8)
    s = (torch.rand(K // G, N, generator=g) * (0.02 - 0.001) + 0.001).half().numpy()
    z = torch.randint(0, 16, (K // G, N), generator=g, dtype=torch.int32).numpy().astype(np.uint8)
    return A, q, s, z
