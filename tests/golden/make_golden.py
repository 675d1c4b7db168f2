"""Write tests/golden/layouts.json: fixed vectors for the synthetic layouts.

The reference ships no golden files or seeded layouts (its benchmark fills
0xAB and never checks data), so these fixtures are generated from the oracle
and serve as regression pins; the oracle itself is pinned independently in
tests/test_oracle.py (Marsaglia's published xorshift64 outputs, brute force,
the reference examples' known-answer byte patterns).

Run from the repo root:  python tests/golden/make_golden.py
"""
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import oracle  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "layouts.json")

# name -> (num_tokens, token_size); stride is always 2 * token_size
LAYOUTS = {
    "cpu_parallel_gather_256x4KB": (256, 4096),
    "small_2048x512B": (2048, 512),
    "small_2048x1KB": (2048, 1024),
    "small_2048x2KB": (2048, 2048),
    "ragged_97x1000B": (97, 1000),
    "direct_8192x4KB": (8192, 4096),
    "kv_2048x64KB": (2048, 65536),
}


def layout_record(n, t):
    stride = 2 * t
    region = np.empty(n * stride, dtype=np.uint8)
    oracle.fill_tokens(region, n, t, stride)
    perm = oracle.permutation(n)
    out = oracle.expected_gather(region, perm, t, stride)
    return {
        "num_tokens": n,
        "token_size": t,
        "stride": stride,
        "perm_head": [int(x) for x in perm[:32]],
        "perm_fnv1a64": "%016x" % oracle.fnv1a64(perm),
        "region_fnv1a64": "%016x" % oracle.fnv1a64(region),
        "token0_fnv1a64": "%016x" % oracle.fnv1a64(region[:t]),
        "output_fnv1a64": "%016x" % oracle.fnv1a64(out),
    }


def kat_direct_transfer():
    """examples/02_direct_transfer.cu:50-54 pattern: 1024 tokens x 4 KB at 2x
    stride, token i filled with i & 0xFF, gathered in order."""
    n, t = 1024, 4096
    out = np.repeat((np.arange(n) & 0xFF).astype(np.uint8), t)
    return {"num_tokens": n, "token_size": t, "output_fnv1a64": "%016x" % oracle.fnv1a64(out)}


def moe_record(tokens=4096, experts=64):
    logits = oracle.moe_logits(tokens, experts)
    top2 = oracle.moe_top2(logits)
    offsets, rows = oracle.moe_lists(top2, experts)
    return {
        "num_tokens": tokens,
        "num_experts": experts,
        "logits_head": [float(x) for x in logits[0, :8]],
        "top2_head": [[int(a), int(b)] for a, b in top2[:8]],
        "expert_counts": [int(x) for x in np.diff(offsets)],
        "rows_fnv1a64": "%016x" % oracle.fnv1a64(rows.astype(np.int32)),
    }


def main():
    rec = {
        "seeds": {
            "data": "%016x" % oracle.DATA_SEED,
            "perm": "%016x" % oracle.PERM_SEED,
            "logits": "%016x" % oracle.LOGITS_SEED,
        },
        "xorshift_head": {
            name: ["%016x" % int(x) for x in oracle.xorshift64_seq(seed, 8)]
            for name, seed in (("data", oracle.DATA_SEED), ("perm", oracle.PERM_SEED),
                               ("logits", oracle.LOGITS_SEED))
        },
        "layouts": {k: layout_record(*v) for k, v in LAYOUTS.items()},
        "kat_direct_transfer": kat_direct_transfer(),
        "moe_4096x64": moe_record(),
    }
    with open(OUT, "w") as f:
        json.dump(rec, f, indent=1, sort_keys=True)
    print("wrote", OUT)


if __name__ == "__main__":
    main()
