"""Writes tests/golden/golden.json — the committed fixtures of the quantized GEMM
parity tests.  Run from the repository root: `python tests/golden/make_golden.py`.

Contents (all data, no code):
  splitmix64  the published SplitMix64 test vector (seed 1234567), which the
              oracle's generator must reproduce;
  kat64       the reference GEMM test's closed-form case
              (flash-kernel-engine tests/test_quantized_gemm.cu:19-48:
              A[i]=(i%7)-3, B[i]=(i%5)-2, B stored [N,K], sa=0.05, sb=0.02),
              evaluated here with numpy int64 arithmetic, independently of the
              C oracle;
  e4m3        the 256-entry E4M3 decode table (fp32 bit patterns) from the OCP
              closed form with exact powers of two, with the reference's
              0x7F/0xFF -> 0.0 rule (src/quantized_gemm.cu:81-97);
  c1          the CPU-sized config (M=128 N=128 K=256, seeded uniform int8,
              per-row/per-column scales U[0.001,0.02]): SHA-256 of the seeded
              inputs and of the oracle's int32 / fp32 / bf16 outputs, plus
              sampled entries.
"""
import hashlib
import json
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

from oracle import oracle as o  # noqa: E402

C1 = dict(M=128, N=128, K=256, seed_A=0xC1A0, seed_B=0xC1B0, seed_sa=0xC15A, seed_sb=0xC15B)


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def c1_inputs():
    M, N, K = C1["M"], C1["N"], C1["K"]
    A = o.gen_i8_uniform((M, K), C1["seed_A"])
    B = o.gen_i8_uniform((N, K), C1["seed_B"])
    sa = o.gen_f32_uniform((M,), C1["seed_sa"], 0.001, 0.02)
    sb = o.gen_f32_uniform((N,), C1["seed_sb"], 0.001, 0.02)
    return A, B, sa, sb


def e4m3_closed_form(code: int) -> float:
    s = -1.0 if code & 0x80 else 1.0
    e, m = (code >> 3) & 0xF, code & 7
    if e == 0:
        return s * m * 2.0 ** -9
    if e == 15 and m == 7:
        return 0.0
    return s * math.ldexp(1.0 + m / 8.0, e - 7)


def main():
    out = {}
    out["splitmix64"] = {"seed": 1234567,
                         "first5": [6457827717110365317, 3203168211198807973, 9817491932198370423,
                                    4593380528125082431, 16408922859458223821]}

    M = N = K = 64
    A = (np.arange(M * K) % 7 - 3).astype(np.int64).reshape(M, K)
    B = (np.arange(N * K) % 5 - 2).astype(np.int64).reshape(N, K)
    acc = A @ B.T
    alpha = np.float32(0.05) * np.float32(0.02)
    out["kat64"] = {
        "M": M, "N": N, "K": K, "sa": 0.05, "sb": 0.02,
        "acc_sum": int(acc.sum()), "acc_min": int(acc.min()), "acc_max": int(acc.max()),
        "acc_nonzero": int((acc != 0).sum()), "acc_row0_first8": acc[0, :8].tolist(),
        "acc_63_63": int(acc[63, 63]),
        "alpha_bits": int(np.array(alpha, dtype=np.float32).view(np.uint32)),
        "acc_sha256": sha(acc.astype(np.int32)),
    }

    out["e4m3"] = [int(np.array(e4m3_closed_form(c), dtype=np.float32).view(np.uint32))
                   for c in range(256)]

    A, B, sa, sb = c1_inputs()
    acc = o.w8a8_acc(A, B)
    f32 = o.w8a8_epilogue(acc, sa, sb, out_dtype=o.OUT_F32)
    bf16 = o.w8a8_epilogue(acc, sa, sb, out_dtype=o.OUT_BF16)
    rng = np.random.default_rng(7)
    idx = rng.integers(0, [C1["M"], C1["N"]], size=(16, 2))
    out["c1"] = dict(C1)
    out["c1"]["sha256"] = {"A": sha(A), "B": sha(B), "scale_a": sha(sa), "scale_b": sha(sb),
                           "acc": sha(acc), "f32": sha(f32), "bf16": sha(bf16)}
    out["c1"]["samples"] = [[int(m), int(n), int(acc[m, n]), int(f32[m:m + 1, n].view(np.uint32)[0]),
                             int(bf16[m, n])] for m, n in idx]

    path = os.path.join(HERE, "golden.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print("wrote", path)


if __name__ == "__main__":
    main()
