"""Writes tests/golden/x4_reference_vectors.json from the reference itself.

Sources, both compiled from the reference's sources by `make -C oracle ref`:
  * oracle/_ref/x4b_host_reference -- cuda/x4b_host_reference.cpp unchanged:
    the order-2^33 root and a 32-point X4 NTT of 11 coefficients
    ((17 i + 3, i^2 + 5), i < 11), the vectors the reference diffs against its
    Rust twin (scripts/check_x4b_cuda_host_reference.sh);
  * oracle/_ref/libx4b_ref.so -- direct_fold_reference of cuda/volta_x4b.cuh:
    codeword folds of the inputs and challenges the reference's X4c host check
    uses (scripts/check_x4c_cuda_host_reference.sh, `symbol` and
    `check_fold_length`), kept whole for input lengths 2..64 and as a SHA-256
    of the output bytes for 2^10 and 2^12.

Run from the repository root where /root/reference exists:
    python3 tests/golden/make_x4_golden.py
"""
import ctypes
import hashlib
import json
import pathlib
import subprocess

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[2]
P = 0xFFFF_FFFF_0000_0001
CHALLENGES = [(0, 0), (1, 0), (3, 11), (P - 1, P - 2)]


def fold_input(n):
    # symbol(index) of the X4c host check
    return np.array([[(i * 0x1_0000_01B3 + 17) & (2**64 - 1), i * i * 97 + i * 19 + 29] for i in range(n)],
                    dtype=np.uint64)


def main():
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "ref"], check=True)
    text = subprocess.run([str(ROOT / "oracle/_ref/x4b_host_reference")], check=True,
                          capture_output=True, text=True).stdout
    vals = dict(line.split("=", 1) for line in text.splitlines() if "=" in line)
    pair = lambda s: [int(h, 16) for h in s.split(":")]
    ntt = [pair(vals["ntt_%02d" % i]) for i in range(32)]
    lib = ctypes.CDLL(str(ROOT / "oracle/_ref/libx4b_ref.so"))
    lib.ref_x4_direct_fold.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_uint64,
                                       ctypes.c_void_p]
    folds = []
    for bits in [1, 2, 3, 4, 5, 6, 10, 12]:
        x = fold_input(1 << bits)
        for ch in CHALLENGES:
            out = np.zeros((x.shape[0] // 2, 2), np.uint64)
            assert lib.ref_x4_direct_fold(x.ctypes.data, x.shape[0], ch[0], ch[1], out.ctypes.data) == 0
            rec = {"bits": bits, "challenge": list(ch)}
            if bits <= 6:
                rec["output"] = out.tolist()
            else:
                rec["sha256"] = hashlib.sha256(out.tobytes()).hexdigest()
            folds.append(rec)
    doc = {
        "source": "oracle/_ref built from cuda/x4b_host_reference.cpp and cuda/volta_x4b.cuh",
        "root_2_33": pair(vals["root_2_33"]),
        "ntt32": {"coefficients": [[i * 17 + 3, i * i + 5] for i in range(11)], "n": 32, "output": ntt},
        "fold_input": "symbol(i) = (i * 0x1000001b3 + 17, 97 i^2 + 19 i + 29)",
        "folds": folds,
    }
    path = ROOT / "tests/golden/x4_reference_vectors.json"
    path.write_text(json.dumps(doc, separators=(",", ":")) + "\n")
    print("wrote", path, path.stat().st_size, "bytes")


if __name__ == "__main__":
    main()
