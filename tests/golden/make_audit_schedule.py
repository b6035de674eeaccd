"""Writes ``zimage_audit_schedule.json`` from the reference's generated
``internal/prometheus/models/zimage-turbo/resolved_audit_schedule.h`` (read as
text, nothing executed): per stage of the NoiseRefiner and ContextRefiner
static-audit schedules the stage id, capture policy (1 full copy, 4 summary
record), element count, arena byte offset and projection keys.  These define
the arena an auditor reads, so the library's records are checked against them.

Run from the repository root with the reference tree at /root/reference."""
import json
import re
import sys
from pathlib import Path

HEADER = Path("/root/reference/internal/prometheus/models/zimage-turbo/resolved_audit_schedule.h")
OUT = Path(__file__).resolve().parent / "zimage_audit_schedule.json"


def _array(text, name):
    body = re.search(rf"{name}\[\]\s*=\s*\{{(.*?)\}};", text, re.S).group(1)
    return body


def _schedule(text, prefix):
    keys = [int(v) for v in re.findall(r"(\d+)u", _array(text, f"k_prom_zimage_turbo_{prefix}projection_keys"))]
    rows = []
    for entry in re.findall(r"\{PROM_ZIMAGE_TURBO_AUDIT_LOCK_ID,([^}]*)\}", _array(text, f"k_prom_zimage_turbo_{prefix}schedule")):
        f = [int(v.strip().rstrip("u")) for v in entry.split(",")]
        stage, policy, source, layout, base, count, koff, kcount, dest = f[:9]
        rows.append({"stage": stage, "policy": policy, "count": count, "dest": dest,
                     "keys": keys[koff:koff + kcount]})
    return rows


def main():
    text = HEADER.read_text()
    define = lambda n: int(re.search(rf"#define {n} (\d+)u", text).group(1))
    data = {
        "noise": {"arena_bytes": define("PROM_ZIMAGE_TURBO_AUDIT_ARENA_BYTES"),
                  "required_bytes": define("PROM_ZIMAGE_TURBO_AUDIT_REQUIRED_BYTES"),
                  "witness_offset": define("PROM_ZIMAGE_TURBO_AUDIT_TRANSIENT_ATTENTION_OFFSET"),
                  "stages": _schedule(text, "audit_")},
        "context": {"arena_bytes": define("PROM_ZIMAGE_TURBO_CONTEXT_AUDIT_ARENA_BYTES"),
                    "required_bytes": define("PROM_ZIMAGE_TURBO_CONTEXT_AUDIT_REQUIRED_BYTES"),
                    "witness_offset": define("PROM_ZIMAGE_TURBO_CONTEXT_AUDIT_TRANSIENT_ATTENTION_OFFSET"),
                    "stages": _schedule(text, "context_audit_")},
    }
    OUT.write_text(json.dumps(data, indent=1) + "\n")
    print(f"wrote {OUT}: {len(data['noise']['stages'])} + {len(data['context']['stages'])} stages")


if __name__ == "__main__":
    sys.exit(main())
