"""The run ledger's fingerprint chain (src/scheduler.cpp:15-24, 280) on the CPU:
FNV-1a known answers, and the fingerprints of the reference's own recorded runs
(tests/golden/fingerprints.json, copied from reports/g1 by make_fingerprints.py)
recomputed from their tokens and logit bits."""
import json
import os

from stride_amd import cli, engine

HERE = os.path.dirname(os.path.abspath(__file__))


def test_fnv1a_known_answers():
    # published 64-bit FNV-1a vectors: "" -> offset basis, "a", "foobar"
    assert engine.fnv_bytes(engine.FNV_OFFSET, b"") == 0xCBF29CE484222325
    assert engine.fnv_bytes(engine.FNV_OFFSET, b"a") == 0xAF63DC4C8601EC8C
    assert engine.fnv_bytes(engine.FNV_OFFSET, b"foobar") == 0x85944171F73967E8
    assert engine.fnv_mix(engine.FNV_OFFSET, 0x64636261) == engine.fnv_bytes(engine.FNV_OFFSET, b"abcd")


def test_reference_run_fingerprints():
    with open(os.path.join(HERE, "golden", "fingerprints.json")) as f:
        recs = json.load(f)
    assert len(recs) >= 4
    for r in recs:
        values = [int(v, 16) for v in r["values"]]
        assert cli.hex64(cli.fingerprint(r["tokens"], values)) == r["fingerprint"], (r["source"], r["id"])
        assert all(cli.hex32(v) == h for v, h in zip(values, r["values"]))


def test_hex_formats():
    assert cli.hex32(0x3F800000) == "3f800000" and cli.hex32(-1) == "ffffffff"
    assert cli.hex64(engine.FNV_OFFSET) == "cbf29ce484222325"
