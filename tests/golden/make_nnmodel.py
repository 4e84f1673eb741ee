"""Writes the small model-file fixtures under tests/golden/ (run: python tests/golden/make_nnmodel.py).

The byte layout follows the reference's model_serialization.hpp (neuralnet-cpp-dev/neuralnet.cpp
v1.18.0): header :38-82 and :500-546, param entry :579-590 / :640-700, save order :999-1073,
per-entry precision tags src/precision_type_test.cpp:388-392. Weights come from the CPU oracle
(absmean tau, trit_pack), so the fixtures do not depend on the library under test.

Model of every fixture: RMSNorm(48) -> BitLinear(48 -> 20) -> BitLinear(20 -> 12), i.e. the entries
  0 gamma (48, 1) Dense | 1 W1 (20, 48) ternary | 2 b1 (20, 1) Dense | 3 W2 (12, 20) ternary | 4 b2 (12, 1) Dense
Files:
  nnmodel_v8.nnmodel        v8, Model role, TernaryPacked2 rows of whole words, sha256 tail
  nnmodel_v7.nnmodel        v7 (no training-state length, no tail), same entries
  nnmodel_trim_f16.nnmodel  v8, gamma as f16, W2 rows trimmed to ceil(K/4) bytes
  nnmodel_ckpt.nnmodel      v8, Checkpoint role, ternary weights as TernaryLatent (f32 latents)
  nnmodel_packed3.nnmodel   v8, W1 as TernaryPacked3 (ceil(K/5) bytes per row; refused by the loader)
  nnmodel_corrupt.nnmodel   nnmodel_v8 with one payload byte flipped (checksum mismatch)
"""
import hashlib
import os
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import nn_oracle as orc  # noqa: E402

MAGIC = 0x4E4E4E4E
DENSE, LATENT, PACKED2, PACKED3 = 0, 1, 2, 3
TAG_F32, TAG_F16 = 0, 2
SPEC = b"spec-bytes: opaque to the loader"
TOKENIZER = b"NNVC-tokenizer-bytes"


def entry(kind, tag, rows, cols, aux=b"", payload=b""):
    return struct.pack("<BBQQQQ", kind, tag, rows, cols, len(aux), len(payload)) + aux + payload


def weights():
    gamma = orc.fill_normal(48, 0xB17A0101, 1.0, 0.1).reshape(48, 1)
    W1 = orc.fill_normal(20 * 48, 0xB17A0102, 0.0, 0.02).reshape(20, 48)
    W2 = orc.fill_normal(12 * 20, 0xB17A0103, 0.0, 0.02).reshape(12, 20)
    b1 = orc.fill_normal(20, 0xB17A0104, 0.0, 0.1).reshape(20, 1)
    b2 = orc.fill_normal(12, 0xB17A0105, 0.0, 0.1).reshape(12, 1)
    return gamma, W1, b1, W2, b2


def packed2(W, trim=False):
    tau = orc.row_absmean(W)
    wq = orc.trit_pack(W, tau)
    rows, K = W.shape
    raw = wq.astype("<u4").tobytes()
    if trim:
        per = (K + 3) // 4
        whole = wq.shape[1] * 4
        raw = b"".join(raw[r * whole:r * whole + per] for r in range(rows))
    return entry(PACKED2, TAG_F32, rows, K, tau.astype("<f4").tobytes(), raw)


def dense(a, tag=TAG_F32):
    rows, cols = a.shape
    data = a.astype("<f4").tobytes() if tag == TAG_F32 else a.astype("<f2").tobytes()
    return entry(DENSE, tag, rows, cols, b"", data)


def file_bytes(version, role, entries):
    out = struct.pack("<IIBB", MAGIC, version, 0, role)
    out += struct.pack("<Q", len(SPEC)) + SPEC
    if version >= 8:
        out += struct.pack("<Q", 0)  # no training-state section
    out += b"".join(entries)
    out += struct.pack("<Q", len(TOKENIZER)) + TOKENIZER
    if version >= 8:
        out += hashlib.sha256(out).digest() + b"NNEND"
    return out


def main(out_dir=HERE):
    gamma, W1, b1, W2, b2 = weights()
    std = [dense(gamma), packed2(W1), dense(b1), packed2(W2), dense(b2)]
    files = {
        "nnmodel_v8.nnmodel": file_bytes(8, 0, std),
        "nnmodel_v7.nnmodel": file_bytes(7, 0, std),
        "nnmodel_trim_f16.nnmodel": file_bytes(8, 0, [dense(gamma, TAG_F16), packed2(W1), dense(b1),
                                                      packed2(W2, trim=True), dense(b2)]),
        "nnmodel_ckpt.nnmodel": file_bytes(8, 1, [dense(gamma), entry(LATENT, TAG_F32, 20, 48, b"", W1.astype("<f4").tobytes()),
                                                  dense(b1), entry(LATENT, TAG_F32, 12, 20, b"", W2.astype("<f4").tobytes()),
                                                  dense(b2)]),
        "nnmodel_packed3.nnmodel": file_bytes(8, 0, [dense(gamma),
                                                     entry(PACKED3, TAG_F32, 20, 48, orc.row_absmean(W1).astype("<f4").tobytes(),
                                                           bytes(20 * ((48 + 4) // 5))),
                                                     dense(b1), packed2(W2), dense(b2)]),
    }
    corrupt = bytearray(files["nnmodel_v8.nnmodel"])
    corrupt[len(corrupt) // 2] ^= 0x01
    files["nnmodel_corrupt.nnmodel"] = bytes(corrupt)
    for name, data in files.items():
        with open(os.path.join(out_dir, name), "wb") as f:
            f.write(data)
        print(name, len(data))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else HERE)
