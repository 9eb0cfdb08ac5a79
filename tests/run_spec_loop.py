"""The full single-GPU speculative configuration with oracle checks.

512 requests, prompts U[128, 1024], 128 generated tokens each, random-init
Qwen3-0.6B draft (batch 64) + Qwen3-8B target (batch 16), depth 4, greedy.
Every 64th forward's mid-depth attention layer call is checked against the
oracle.  Prints one progress line per round and a JSON summary last; exits
nonzero if a check fails.  Usage: python tests/run_spec_loop.py [--requests N]
"""

from __future__ import annotations

import argparse
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [HERE, os.path.dirname(HERE)]

from nebulasd_amd.spec_loop import run  # noqa: E402
from spec_checks import make_checker  # noqa: E402


def main():
    p = argparse.ArgumentParser()
    p.add_argument("--requests", type=int, default=512)
    p.add_argument("--new-tokens", type=int, default=128)
    p.add_argument("--check-every", type=int, default=64)
    a = p.parse_args()
    results = []
    res = run(n_requests=a.requests, new_tokens=a.new_tokens, check_every=a.check_every,
              make_check=make_checker(results), log=lambda m: print(m, flush=True))
    res["checks_ok"] = all(r["ok"] for r in results)
    res["checks"] = len(results)
    res["worst_check"] = max(results, key=lambda r: r["excess_o"]) if results else None
    res["worst_dlse"] = max((r["max_dlse"] for r in results), default=None)
    print(json.dumps(res), flush=True)
    sys.exit(0 if res["checks_ok"] and results else 1)


if __name__ == "__main__":
    main()
