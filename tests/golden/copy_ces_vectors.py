"""Copy a subset of the reference's committed SSD golden vectors into this directory.

The vectors are data that the reference ships beside its own verifier
(stream/ces/ssd_reference/golden_vectors/*.npz, checked by
stream/ces/ssd_reference/verify.py:26 at max-abs 1e-5). They are copied
byte-for-byte; no reference code is run or copied. Each file holds fp32
arrays x (B,T,H), A (H,), B, C (B,T,H,N), dt (B,T,H), D (H,), dt_bias (H,),
expected_y (B,T,H) and a JSON metadata string.

Run once in a container that has /root/reference mounted:
    python tests/golden/copy_ces_vectors.py
"""
import shutil
from pathlib import Path

SRC = Path("/root/reference/stream/ces/ssd_reference/golden_vectors")
DST = Path(__file__).resolve().parent / "ces"
NAMES = [f"ssd_B2_T128_H4_N16_seed{s}.npz" for s in range(42, 52)] + [
    "ssd_B2_T512_H4_N16_seed52.npz",
    "ssd_B2_T512_H4_N16_seed53.npz",
    "ssd_B2_T2048_H4_N16_seed62.npz",
]

if __name__ == "__main__":
    DST.mkdir(exist_ok=True)
    for n in NAMES:
        shutil.copyfile(SRC / n, DST / n)
        print("copied", n)
