"""Writes tests/golden/config_inputs.json: for each benchmark configuration,
the SHA-256 of its packed input buffer (little-endian bytes, row-major), its
shape, dtype and first/last elements, and the same for the challenges.

    python tests/golden/make_config_inputs.py

The inputs come from volta_mi355x.workloads (C1's rows from the oracle's
FpStream restatement, the generator the device's ChaCha8 rows reproduce).
tests/test_config_fixtures.py recomputes every entry except the full C4 and C5
buffers (4 GiB of lanes and 8 GiB): for those it checks the leading-row
entries, which pin the same streams (numpy draws them element by element).
"""
from __future__ import annotations

import hashlib
import json
import pathlib
import sys

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT / "volta-zk_amd"), str(ROOT / "oracle")]
OUT = pathlib.Path(__file__).resolve().parent / "config_inputs.json"


def fingerprint(a: np.ndarray) -> dict:
    a = np.ascontiguousarray(a)
    flat = a.reshape(-1)
    return {"shape": list(a.shape), "dtype": str(a.dtype), "sha256": hashlib.sha256(a.tobytes()).hexdigest(),
            "first": int(flat[0]), "last": int(flat[-1])}


def generators():
    """(name, zero-argument generator) for every fingerprinted buffer."""
    import oracle
    from volta_mi355x import workloads as W
    c1 = W.CONFIGS["c1"]
    yield "c1/rows", lambda: oracle.fp_rows(W.SEED_C1_ROWS, 0, c1.rows, c1.msg_len)
    yield "c1/challenges", lambda: W.uniform_fp("volta-mi355x/c1/challenges", c1.rows)
    yield "c2/weights", W.c2_weights
    yield "c2/challenges", lambda: W.challenges_fp2("volta-mi355x/c2/challenges", 2)
    yield "c3/weights", W.c3_weights
    yield "c3/challenges", lambda: W.challenges_fp2("volta-mi355x/c3/challenges", 2)
    yield "c4/messages", W.c4_messages
    yield "c4/messages[:256]", lambda: W.c4_messages(rows=256)
    yield "c5/rows", W.c5_rows
    yield "c5/rows[:1]", lambda: W.c5_rows(rows=1)
    yield "c5/challenges", lambda: W.challenges_fp2("volta-mi355x/c5/challenges", 1)
    yield "c5/queries", lambda: W.c5_query_columns(1 << 24, 256)
    for name in ("p15", "p17"):
        cfg = W.CONFIGS[name]
        yield f"{name}/weights", (lambda cfg=cfg, name=name:
                                  W.gaussian_i16(f"volta-mi355x/{name}/weights", cfg.rows * cfg.msg_len))


def main() -> None:
    out = {}
    for name, gen in generators():
        out[name] = fingerprint(gen())
        print(name, out[name]["sha256"][:16], flush=True)
    OUT.write_text(json.dumps(out, indent=1, sort_keys=True) + "\n")


if __name__ == "__main__":
    main()
