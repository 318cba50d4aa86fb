"""Extract boundary events from the reference's decode archive into a small JSON fixture.

The archive ``gpt-oss-20b/runs/perhead/decode/trials-000.jsonl.gz`` holds, per
trial, the policy config and the per-boundary events the runtime wrote
(R:494-496: boundary, before, after, freed, swa_cursor). They pin the count
arithmetic of the boundary (before = resident, after = budget or P+R, freed =
before - after) on real runs. Reads data only; runs no reference code.

Usage: python tests/golden/make_archive_events.py [/root/reference]
"""
import gzip
import json
import sys
from pathlib import Path

root = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
src = root / "gpt-oss-20b/runs/perhead/decode/trials-000.jsonl.gz"
out = []
seen = set()
with gzip.open(src, "rt") as f:
    for line in f:
        r = json.loads(line)
        cfg = r["policy"]
        key = (cfg["name"], cfg["budget"])
        if key in seen or not any(e.get("freed") for e in r["events"]):
            continue
        seen.add(key)
        events = [{k: e[k] for k in ("boundary", "before", "after", "freed", "swa_cursor", "deferred", "protected")
                   if k in e} for e in r["events"]]
        out.append({"policy": cfg, "peak_full_entries": r["peak_full_entries"], "freed": r["freed"],
                    "events": events})
dest = Path(__file__).with_name("archive_events.json")
dest.write_text(json.dumps(out, indent=1) + "\n")
print(f"wrote {len(out)} trials to {dest}")
