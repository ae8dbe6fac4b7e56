"""Writes the committed golden fixtures under tests/golden/.

page16_tiny.npz - BASELINE config 1 (B=4, Hq=32, Hkv=8, D=128, fp16, pool 1024
pages, L ~ U{256..2048}) for seed 1234: sha256 digests of the generated inputs
(so a changed generator is caught), the block table and lengths, and the
closed-form fp64 output of the oracle (dense softmax attention over the
gathered pages).

Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import oracle  # noqa: E402
from unifiedkv_amd import workloads  # noqa: E402

SEED = 1234


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def tiny_fixture():
    case = workloads.numpy_case("tiny", SEED)
    dt = workloads.DTYPE_CODES[case["dtype"]]
    qf = oracle.bits_to_f32(case["q"], dt)
    kf = oracle.bits_to_f32(case["k_cache"], dt)
    vf = oracle.bits_to_f32(case["v_cache"], dt)
    dense = oracle.page16_decode_dense(qf, kf, vf, case["block_table"], case["seqlens"],
                                       softmax_scale=case["scale"], n_rep=case["n_rep"])
    return dict(
        seed=np.int64(SEED),
        q_sha=digest(case["q"]), k_sha=digest(case["k_cache"]), v_sha=digest(case["v_cache"]),
        block_table=case["block_table"], seqlens=case["seqlens"],
        out_f64=dense,
    )


def main():
    out = Path(__file__).resolve().parent / "page16_tiny.npz"
    np.savez_compressed(out, **tiny_fixture())
    print("wrote", out)


if __name__ == "__main__":
    main()
