"""Write the RoPE table fixture: cos/sin of compute_rope_params(head_dim=128,
theta=1e6, context_length=2048) in fp16 (torchpp/dlops/rope.py:43-54, the
tables the Qwen3-shape model and BASELINE config 2 use).

The table comes from the CPU oracle (oracle/ops.py:compute_rope_params), whose
values tests/test_oracle.py pins against an fp64 closed form; the fixture
freezes its exact fp16 bit pattern (SHA-256 of the little-endian uint16 words
of the whole table) plus 64 rows of it, so a change of dtype, ordering or
rounding anywhere on the way to the kernels shows up as a bit difference.

Run from the repository root:  python tests/golden/make_rope_params.py
"""
import hashlib
import json
import os
import sys

import numpy as np

sys.path.insert(0, os.path.abspath(os.path.join(os.path.dirname(__file__), "..", "..")))
import oracle  # noqa: E402

HEAD_DIM, THETA, CTX = 128, 1e6, 2048
ROWS = list(range(32)) + list(range(64, CTX, 64))


def table_bits(t):
    return np.ascontiguousarray(t.numpy().view(np.uint16))


def sha256(bits):
    return hashlib.sha256(bits.astype("<u2").tobytes()).hexdigest()


def main():
    cos, sin = oracle.compute_rope_params(HEAD_DIM, THETA, CTX)
    cb, sb = table_bits(cos), table_bits(sin)
    out = {
        "what": "compute_rope_params(128, 1e6, 2048) fp16 cos/sin (rope.py:43-54)",
        "head_dim": HEAD_DIM, "theta": THETA, "context_length": CTX,
        "sha256_cos": sha256(cb), "sha256_sin": sha256(sb),
        "rows": ROWS,
        "cos_rows_u16": cb[ROWS].tolist(), "sin_rows_u16": sb[ROWS].tolist(),
    }
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "rope_params_d128_t1e6_s2048.json")
    with open(path, "w") as f:
        json.dump(out, f, separators=(",", ":"))
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
