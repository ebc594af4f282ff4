#!/usr/bin/env python3
"""Generates the BASELINE config-5 fixture: a random tensor network of 10
input tensors of rank 4-6, every mode of size 2, 4, 8 or 16, each mode shared
by exactly two tensors or by one tensor and the output, contracted along the
greedy min-size pairing path; the total work is kept near 50 GFLOP.

Writes c5_network.json (einsum string, sizes per mode name, path in
opt_einsum's standard form, FLOP count).  Deterministic for a given seed.
Usage: python tests/golden/make_c5_network.py [seed]
"""
import json
import os
import string
import sys

import numpy as np

LETTERS = string.ascii_lowercase + string.ascii_uppercase


def make_network(rng, n_tensors=10):
    ranks = rng.integers(4, 7, n_tensors)
    slots = [t for t, r in enumerate(ranks) for _ in range(r)]
    n_open = int(rng.integers(3, 6))
    if (len(slots) - n_open) % 2:
        n_open += 1
    for _ in range(1000):
        perm = list(rng.permutation(len(slots)))
        open_slots, rest = perm[:n_open], perm[n_open:]
        pairs = [(slots[rest[i]], slots[rest[i + 1]]) for i in range(0, len(rest), 2)]
        if all(a != b for a, b in pairs):
            break
    else:
        raise RuntimeError("no valid pairing")
    modes = [[] for _ in range(n_tensors)]
    out = []
    m = 0
    for a, b in pairs:
        modes[a].append(LETTERS[m])
        modes[b].append(LETTERS[m])
        m += 1
    for s in open_slots:
        modes[slots[s]].append(LETTERS[m])
        out.append(LETTERS[m])
        m += 1
    sizes = {LETTERS[i]: int(rng.choice([2, 4, 8, 16])) for i in range(m)}
    modes = [list(rng.permutation(x)) for x in modes]
    return modes, out, sizes


def greedy_path(modes, out, sizes):
    """Repeatedly contracts the pair (sharing a mode if possible) whose result
    is smallest; returns the path in standard form and the total FLOP count."""
    live = [list(x) for x in modes]
    path, flops = [], 0
    while len(live) > 1:
        best = None
        for i in range(len(live)):
            for j in range(i + 1, len(live)):
                shared = set(live[i]) & set(live[j])
                rest = [x for k, t in enumerate(live) if k not in (i, j) for x in t] + list(out)
                res = [d for d in dict.fromkeys(live[i] + live[j]) if d in rest]
                size = int(np.prod([sizes[d] for d in res])) if res else 1
                allm = dict.fromkeys(live[i] + live[j])
                f = 2 * int(np.prod([sizes[d] for d in allm]))
                key = (0 if shared else 1, size, f)
                if best is None or key < best[0]:
                    best = (key, i, j, res, f)
        _, i, j, res, f = best
        path.append((i, j))
        flops += f
        live = [t for k, t in enumerate(live) if k not in (i, j)] + [sorted(res)]
    return path, flops


def generate(seed, target=50e9, lo=35e9, hi=70e9):
    rng = np.random.default_rng(seed)
    for _ in range(20000):
        modes, out, sizes = make_network(rng)
        path, flops = greedy_path(modes, out, sizes)
        if lo <= flops <= hi:
            return modes, out, sizes, path, flops
    raise RuntimeError("no network in the FLOP window")


def main():
    seed = int(sys.argv[1]) if len(sys.argv) > 1 else 5
    modes, out, sizes, path, flops = generate(seed)
    expr = ",".join("".join(t) for t in modes) + "->" + "".join(out)
    used = sorted(set(c for c in expr if c.isalpha()))
    fixture = {
        "seed": seed,
        "expr": expr,
        "sizes": {k: sizes[k] for k in used},
        "path": [list(p) for p in path],
        "flops": flops,
        "note": "BASELINE config 5: random tensor network, greedy min-size path",
    }
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c5_network.json")
    with open(dst, "w") as f:
        json.dump(fixture, f, indent=1)
    print(expr, f"{flops / 1e9:.1f} GFLOP", path)


if __name__ == "__main__":
    main()
