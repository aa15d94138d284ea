"""Write golden vectors for the Q4_K / Q6_K block encoders.

Runs ONLY in the build container, where the reference checkout exists: it
imports the reference's own converter (scripts/convert-to-gguf.py, stdlib-only;
its main() is behind `if __name__ == "__main__"`) and records, for seeded inputs,
the exact bytes of q4k_encode_block / q6k_encode_block. The committed output
(kquant_encoder_vectors.npz) is data: inputs and expected outputs.

Usage: python tests/golden/gen_kquant_encoder_vectors.py
"""
import importlib.util
import os
import struct

import numpy as np

REF = "/root/reference/scripts/convert-to-gguf.py"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "kquant_encoder_vectors.npz")


def main():
    spec = importlib.util.spec_from_file_location("ref_convert", REF)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    rng = np.random.default_rng(20260712)
    cases = []
    # Gaussian blocks at several scales, plus edge shapes: all-zero, constant,
    # all-negative, one outlier, tiny values (f16 subnormal scales).
    for scale in (0.02, 1.0, 7.5):
        for _ in range(6):
            cases.append(rng.normal(0.0, scale, 256).astype(np.float32))
    cases.append(np.zeros(256, np.float32))
    cases.append(np.full(256, 0.25, np.float32))
    cases.append(-np.abs(rng.normal(0, 1, 256)).astype(np.float32))
    x = rng.normal(0, 0.01, 256).astype(np.float32)
    x[17] = 3.0
    cases.append(x)
    cases.append((rng.normal(0, 1, 256) * 1e-6).astype(np.float32))
    inputs = np.stack(cases)
    q4k = np.stack([np.frombuffer(mod.q4k_encode_block([float(v) for v in row]), np.uint8) for row in inputs])
    q6k = np.stack([np.frombuffer(mod.q6k_encode_block([float(v) for v in row]), np.uint8) for row in inputs])
    assert q4k.shape[1] == 144 and q6k.shape[1] == 210
    np.savez_compressed(OUT, inputs=inputs, q4k=q4k, q6k=q6k)
    print(f"wrote {OUT}: {len(inputs)} blocks")


if __name__ == "__main__":
    main()
