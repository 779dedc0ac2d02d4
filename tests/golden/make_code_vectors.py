"""Write golden vectors for the trellis codebook functions.

The 1MAD / 3INST / HYB generators are bit-level hash functions: no closed form,
invariant or brute-force check pins their exact output, so their vectors come
from the reference's own numpy implementation (src/codes/ref.py:33-41, :76-91,
:116-127), imported from /root/reference in this container only.  The output
file ``code_vectors.json`` holds data only: SHA-256 digests of the full float32
codebooks at L=16 and a strided sample of states with their values.

Run:  python tests/golden/make_code_vectors.py   (needs /root/reference)
"""
import hashlib
import json
import os
import sys

import numpy as np

REF = "/root/reference"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "code_vectors.json")


def hyb_lut():
    """Deterministic synthetic (512, 2) LUT used for the HYB vectors."""
    return np.random.default_rng(2).standard_normal((512, 2)).astype(np.float32)


def main():
    sys.path.insert(0, REF)
    from src.codes.ref import decode_1mad_batch, decode_3inst_batch, decode_hyb_batch

    L = 16
    states = np.arange(1 << L, dtype=np.uint32)
    sample = np.arange(0, 1 << L, 61, dtype=np.int64)
    lut = hyb_lut()
    books = {
        "1mad": np.asarray(decode_1mad_batch(states), dtype=np.float32).reshape(-1, 1),
        "3inst": np.asarray(decode_3inst_batch(states), dtype=np.float32).reshape(-1, 1),
        "hyb": np.asarray(decode_hyb_batch(states, lut, Q=9), dtype=np.float32).reshape(-1, 2),
    }
    out = {"L": L, "sample_states": sample.tolist(), "hyb_lut_seed": 2, "codes": {}}
    for name, cb in books.items():
        cb = np.ascontiguousarray(cb, dtype=np.float32)
        out["codes"][name] = {
            "V": int(cb.shape[1]),
            "sha256_f32": hashlib.sha256(cb.tobytes()).hexdigest(),
            "sample_bits": cb[sample].view(np.uint32).tolist(),
        }
    with open(OUT, "w") as f:
        json.dump(out, f)
    print("wrote", OUT)


if __name__ == "__main__":
    main()
