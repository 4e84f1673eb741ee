"""Writes tests/golden/matmul_q_i8.npz: seeded inputs and expected outputs of the
trit_pack -> quantize_i8 -> matmul_q_i8 path, produced by the CPU oracle.

The reference ships no fixture files for this path (its golden values are inline KATs, which
tests/test_oracle.py checks directly), and its implementation cannot be built here, so these
fixtures are the oracle's outputs on deterministic inputs (in-repo splitmix64 RNG). They pin
the GPU path and any later change of the oracle to the same numbers.

Cases:
  kat_130x17x6 / kat_512x256x8  the int8_act_test shapes (src/int8_act_test.cpp:483-484),
                                uniform(-1,1) inputs, per-row absmean tau, s = absmax
  c1_1024x1024x8                BASELINE config 0: W ~ N(0,0.02) seed 0xB17A0001, per-tensor
                                absmean tau, X ~ N(0,1) seed 0xB17A0002, s = absmax * fl(1/127)
                                (W itself is not stored: wq is its packed form)

Usage: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import nn_oracle as orc  # noqa: E402


def case_uniform(N, K, M, seed):
    W = orc.fill_uniform(N * K, seed).reshape(N, K)
    tau = np.abs(W.astype(np.float64)).mean(axis=1).astype(np.float32)
    X = orc.fill_uniform(K * M, seed + 1).reshape(K, M)
    s = np.abs(X).max(axis=0).astype(np.float32)
    return W, tau, X, s


def case_c1():
    N = K = 1024
    M = 8
    W = orc.fill_normal(N * K, 0xB17A0001, 0.0, 0.02).reshape(N, K)
    tau = np.full(N, np.abs(W.astype(np.float64)).mean(), np.float32)
    X = orc.fill_normal(K * M, 0xB17A0002, 0.0, 1.0).reshape(K, M)
    s = orc.act_scale(X)
    return W, tau, X, s


def main():
    out = {}
    cases = {
        "kat_130x17x6": case_uniform(130, 17, 6, 31),
        "kat_512x256x8": case_uniform(512, 256, 8, 41),
        "c1_1024x1024x8": case_c1(),
    }
    for name, (W, tau, X, s) in cases.items():
        N, K = W.shape
        M = X.shape[1]
        wq = orc.trit_pack(W, tau)
        xq = orc.quantize_i8(X, s, True)
        acc = orc.matmul_q_i8_acc(wq, xq, K, M)
        Y = orc.matmul_q_i8(wq, tau, xq, s, K, M)
        rec = {"shape": np.array([N, K, M], np.int64), "tau": tau, "X": X, "s": s, "wq": wq,
               "xq": xq, "acc": acc, "Y": Y}
        if N * K <= 4096:
            rec["W"] = W
        for k, v in rec.items():
            out[f"{name}__{k}"] = v
    path = os.path.join(HERE, "matmul_q_i8.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
