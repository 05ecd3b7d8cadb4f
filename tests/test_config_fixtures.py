"""The benchmark configurations' synthetic inputs match the committed
fingerprints in tests/golden/config_inputs.json (SHA-256 of the packed
buffer plus its first and last elements), so a change of generator, seed or
numpy stream is caught on the CPU.  The full C4 and C5 buffers (4 GiB of
lanes, 8 GiB) are checked through their leading rows, drawn from the same
streams."""
import json
import pathlib
import sys

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE / "golden"))

FIXTURES = json.loads((HERE / "golden" / "config_inputs.json").read_text())
SKIP_FULL = {"c4/messages", "c5/rows"}


def test_every_configuration_has_a_fingerprint():
    for key in ("c1/rows", "c2/weights", "c3/weights", "c4/messages", "c5/rows", "p15/weights", "p17/weights"):
        assert key in FIXTURES


def test_inputs_match_fingerprints(oracle):
    import make_config_inputs as M
    seen = set()
    for name, gen in M.generators():
        if name in SKIP_FULL:
            continue
        assert M.fingerprint(gen()) == FIXTURES[name], name
        seen.add(name)
    assert seen == set(FIXTURES) - SKIP_FULL


def test_prefix_rows_are_the_full_buffers_leading_rows():
    """The leading-row fingerprints stand for the full buffers: a smaller
    generator call yields exactly the first rows of the full one."""
    from volta_mi355x import workloads as W
    assert (W.c4_messages(rows=3) == W.c4_messages(rows=5)[:3]).all()
    assert (W.c5_rows(rows=1, n=1 << 10) == W.uniform_fp("volta-mi355x/c5/rows", (3, 1 << 10))[:1]).all()
    assert FIXTURES["c4/messages[:256]"]["first"] == FIXTURES["c4/messages"]["first"]
    assert FIXTURES["c5/rows[:1]"]["first"] == FIXTURES["c5/rows"]["first"]
