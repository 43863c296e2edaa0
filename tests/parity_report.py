#!/usr/bin/env python3
"""Turn the error records the GPU parity tests append to GRINQH_PARITY_LOG
(one JSON object per case) into a markdown table of max abs / rel error per
configuration, against the reference's own semantics and against the product
the serving kernel computes.

    python tests/parity_report.py gpurun_out/parity.jsonl > table.md
"""
import json
import sys


def fmt(v):
    return f"{v:.2e}" if v else "0"


def main(path: str) -> int:
    rows = [json.loads(line) for line in open(path) if line.strip()]
    print("| config | case | rows held | weight rounded | max abs (vs ref) | max rel (vs ref) | "
          "max abs / rms (vs ref) | max abs / rms (vs own) |")
    print("|---|---|---:|:-:|---:|---:|---:|---:|")
    for r in rows:
        ref = r.get("vs_reference", {})
        own = r.get("vs_own", {})
        print(f"| {r['config']} | {r['case']} | {r.get('rows_checked', '')} | "
              f"{'yes' if r.get('weight_rounded') else ('no' if 'weight_rounded' in r else '')} | "
              f"{fmt(ref.get('max_abs', 0))} | {fmt(ref.get('max_rel', 0))} | {fmt(ref.get('max_abs_over_rms', 0))} | "
              f"{fmt(own.get('max_abs_over_rms', 0)) if own else ''} |")
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1]))
