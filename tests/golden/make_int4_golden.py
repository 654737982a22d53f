"""Writes tests/golden/int4_k256_n64_g64.npz: a small seeded INT4 / W4A16 fixture.

The reference holds no INT4 vectors (it has no INT4 code), so this fixture freezes this
library's written specification as produced by the oracle (seed 42): GPTQ packing,
the prepacked layout, packed zeros, fp16 dequantised weights (bit patterns) and the fp32
W4A16 product.  The GPU tests compare the device prepack/unpack against it bit-exactly.

    python tests/golden/make_int4_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import int4 as oi  # noqa: E402


def main() -> None:
    K, N, G, M = 256, 64, 64, 3
    A, q, s, z = oi.make_inputs(M, K, N, G, seed=42)
    qweight = oi.pack_gptq(q)
    out = dict(
        A=A.numpy(), q=q, scales=s, zeros_u8=z, qweight=qweight, packed=oi.prepack(qweight),
        zeros_packed=oi.pack_zeros(z), w_fp16_bits=oi.dequant(q, s, z, G).view(np.uint16),
        Y=oi.w4a16_ref(A, q, s, z, G).numpy(),
    )
    path = os.path.join(HERE, "int4_k256_n64_g64.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
