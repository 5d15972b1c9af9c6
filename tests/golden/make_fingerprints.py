"""Copies a few (tokens, logit bits, fingerprint) records of the reference's own
run ledgers (reports/g1/stride_exact_c1.jsonl and stride_tc_c1.jsonl: real
Llama-3.2-1B greedy runs of the reference's scheduler, src/scheduler.cpp:280)
into fingerprints.json as data, so that the fingerprint chain can be checked
without the reference tree. Run from the repository root with the reference at
/root/reference."""
import json
import sys

src = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/reports/g1"
out = []
for name in ("stride_exact_c1.jsonl", "stride_tc_c1.jsonl"):
    with open(f"{src}/{name}") as f:
        recs = [json.loads(line) for line in f]
    for r in recs[:3]:
        out.append({"source": name, "id": r["id"], "tokens": r["tokens"], "values": r["values"],
                    "fingerprint": r["fingerprint"], "finish": r["finish"]})
with open("tests/golden/fingerprints.json", "w") as f:
    json.dump(out, f)
print(len(out), "records")
