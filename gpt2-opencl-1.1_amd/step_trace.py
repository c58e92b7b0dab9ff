"""Reader of the decode step kernel's phase trace.

With G2_STEP_TRACE=<file> in the environment, the library records, for the
last decode step of a model, the 100 MHz wall clock of every work-group at
each phase boundary of every layer (g2_step.hip, TRACE(k)) and writes them to
<file>: three header words (work-groups, layers, words per work-group), then
per work-group 24 words per layer and 8 for the LM head and the pick.

Usage: python step_trace.py <file> [--heads NH]

Prints the per-phase medians over work-groups and layers 1..L-2, the
per-layer time, and for every hand-off how long after its last producer the
median consumer had the vector (and how far the last producer trailed the
median one).
"""
import argparse
import sys

import numpy as np

# slot -> boundary (g2_step.hip TRACE(k))
SLOTS = {
    0: "layer start (X2 fetch issued)", 1: "X2 in", 11: "LayerNorm 1 done", 12: "qkv dots done",
    2: "q/k/v published", 3: "attention units done", 4: "head merge done", 5: "O in", 6: "X1 published",
    7: "X1 in", 13: "LayerNorm 2 done", 14: "fc dots done", 8: "H published", 9: "H in", 15: "fc2 dots done",
    10: "X2 published", 16: "O published",
}
ORDER = [0, 1, 11, 12, 2, 3, 4, 5, 6, 7, 13, 14, 8, 9, 15, 10]


def load(path):
    d = np.fromfile(path, dtype=np.uint64)
    nwg, L, stride = int(d[0]), int(d[1]), int(d[2])
    raw = d[3:3 + nwg * stride].reshape(nwg, stride).astype(np.int64)
    t = (raw - raw[:, 0].min()) * 10 / 1000.0  # microseconds
    return nwg, L, t


def summary(path, heads):
    nwg, L, t = load(path)
    f = t[:, :24 * L].reshape(nwg, L, 24)
    mid = slice(1, L - 1)
    out = [f"work-groups {nwg}, layers {L}; step {t[0, 24 * L + 2]:.1f} us (work-group 0's pick), "
           f"LM head in {np.median(t[:, 24 * L]):.1f}, done {np.median(t[:, 24 * L + 1]):.1f}"]
    per_layer = np.median(f[:, 2:, 0] - f[:, 1:-1, 0], axis=0)
    out.append(f"per-layer time (median over work-groups and layers): {np.median(per_layer):.2f} us")
    out.append("phase (median over work-groups, layers 1..L-2), us:")
    for a, b in zip(ORDER, ORDER[1:]):
        rows = slice(None)
        if a in (4, 5) or b in (4, 5):
            rows = slice(heads, None)  # work-groups that merge no head
        d = np.median(f[rows, mid, b] - f[rows, mid, a])
        out.append(f"  {SLOTS[a]:30s} -> {SLOTS[b]:30s} {d:6.2f}")
    nxt = np.median(f[:, 2:L - 1, 0] - f[:, 1:L - 2, 10])
    out.append(f"  {SLOTS[10]:30s} -> {'next layer start':30s} {nxt:6.2f}")
    hops = [("X2 -> qkv", 10, 1, slice(None), 1), ("q/k/v -> attention", 2, 3, slice(None), 0),
            ("O -> proj", 16, 5, slice(0, heads), 0), ("X1 -> fc", 6, 7, slice(heads, None), 0),
            ("H -> fc2", 8, 9, slice(None), 0)]
    # the merging work-groups: their attention units, then the wait for the
    # head's other chunk partials and the merge, up to O published
    m = f[:heads, mid]
    out.append(f"head-merging work-groups (median): attention units done -> O published "
               f"{np.median(m[..., 16] - m[..., 3]):.2f} us; last attention unit of any work-group -> "
               f"O published {np.median(f[:heads, mid, 16] - f[:, mid, 3].max(axis=0)):.2f} us")
    out.append("hand-offs (median consumer in - last producer's publish | last - median producer), us:")
    for name, ps, cs, prod, prev in hops:
        lat, skew = [], []
        for l in range(2, L - 1):
            pub = f[prod, l - prev, ps]
            cons = f[heads:, l, cs] if cs == 5 else f[:, l, cs]
            lat.append(np.median(cons - pub.max()))
            skew.append(pub.max() - np.median(pub))
        out.append(f"  {name:20s} {np.median(lat):6.2f} | {np.median(skew):5.2f}")
    return "\n".join(out)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("trace")
    ap.add_argument("--heads", type=int, default=25, help="n_head of the model (head-merging work-groups)")
    args = ap.parse_args(argv)
    print(summary(args.trace, args.heads))
    return 0


if __name__ == "__main__":
    sys.exit(main())
