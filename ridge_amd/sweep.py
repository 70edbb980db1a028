"""Registered sweep shapes for the MI355X ground-truth measurement.

    python -m ridge_amd.sweep [--seed S] [--out data/sweep/mi355x-registered.csv]

The reference registers 14 hand-picked A100 shapes before measuring anything
(data/sweep/phase4-registered.csv:1-52). Here the 14 shapes are drawn from a
fixed seed: M and N from {1024, 2048, 4096, 8192, 16384}, K from
{128, 1024, 4096, 8192} (or the sets --mn-values and --k-values give), element i
of the draw being splitmix64(seed, i) modulo the set size (three draws per
shape, duplicates and excluded shapes redrawn). Every M and N is a multiple of
256 and every K of 128, so every registered variant divides every shape; a space
with too few new shapes left is refused. The file is written once and committed before the first measurement;
changing it afterwards is a visible, separate commit.
"""

import argparse
import os

MN_CHOICES = (1024, 2048, 4096, 8192, 16384)
K_CHOICES = (128, 1024, 4096, 8192)
DEFAULT_SEED = 0x5EED2026
M64 = (1 << 64) - 1


def splitmix64_at(seed, i):
    z = (seed + (i + 1) * 0x9E3779B97F4A7C15) & M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def registered_shapes(seed=DEFAULT_SEED, count=14, exclude=(), mn_choices=MN_CHOICES, k_choices=K_CHOICES):
    """`count` distinct shapes drawn in order; a draw already taken, or listed in
    `exclude` (the shapes of another registered sweep, for a held-out set),
    is redrawn. Refuses a space with fewer than `count` shapes left to draw."""
    if any(v % 256 for v in mn_choices) or any(v % 128 for v in k_choices) or min(k_choices) < 128:
        raise ValueError("every M and N must be a multiple of 256 and every K of 128 (at least 128), so that "
                         "every row of the kernel table divides every shape")
    left = {(M, N, K) for M in mn_choices for N in mn_choices for K in k_choices} - set(exclude)
    if len(left) < count:
        raise ValueError("the shape space holds %d shapes outside the excluded sets, %d needed" % (len(left), count))
    shapes, i = [], 0
    while len(shapes) < count:
        M = mn_choices[splitmix64_at(seed, i) % len(mn_choices)]
        N = mn_choices[splitmix64_at(seed, i + 1) % len(mn_choices)]
        K = k_choices[splitmix64_at(seed, i + 2) % len(k_choices)]
        i += 3
        if (M, N, K) not in shapes and (M, N, K) not in exclude:
            shapes.append((M, N, K))
    return shapes


def rationale(M, N, K):
    tiles = (M // 256) * (N // 256)
    return ("%d workgroups at 256x256 = %.2f waves over 256 CUs; %d K-tiles at BK=64; "
            "%.1f FLOP/B compulsory" % (tiles, tiles / 256.0, K // 64,
                                        2.0 * M * N * K / (2.0 * (M * K + K * N + M * N))))


# The BASELINE.json configs measured beside the sweep (not part of the regret set).
BASELINE_SHAPES = [
    (1024, 1024, 1024, "baseline-1024cube"),
    (4096, 4096, 4096, "baseline-4096cube-headline"),
    (8192, 8192, 128, "baseline-small-k"),
    (16384, 128, 8192, "baseline-tall-skinny"),
]


def write_registered(path, seed=DEFAULT_SEED, prefix="s", exclude=(), note=(), mn_choices=MN_CHOICES,
                     k_choices=K_CHOICES):
    shapes = registered_shapes(seed, exclude=exclude, mn_choices=mn_choices, k_choices=k_choices)
    lines = [
        "# MI355X registered sweep: 14 shapes drawn by ridge_amd/sweep.py with seed 0x%X." % seed,
        "# Registered before any measurement. The tile configs are the kernel table",
        "# (ridge_amd/csrc/gemm_variants.def); the sweep is every shape x every variant.",
    ] + ["# " + n for n in note] + ["# M,N,K,tag,rationale"]
    for i, (M, N, K) in enumerate(shapes):
        lines.append("%d,%d,%d,%s%02d-%dx%dx%d,%s" % (M, N, K, prefix, i, M, N, K, rationale(M, N, K)))
    with open(path, "w") as f:
        f.write("\n".join(lines) + "\n")


def write_baseline(path):
    lines = ["# BASELINE.json configs, measured over the variants that divide each.", "# M,N,K,tag,rationale"]
    for M, N, K, tag in BASELINE_SHAPES:
        lines.append("%d,%d,%d,%s,%s" % (M, N, K, tag, rationale(M, N, K) if N >= 256 else
                                         "N=128: one column of 128-wide tiles, A streamed once"))
    with open(path, "w") as f:
        f.write("\n".join(lines) + "\n")


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--seed", type=lambda s: int(s, 0), default=DEFAULT_SEED)
    ap.add_argument("--out", default="data/sweep/mi355x-registered.csv")
    ap.add_argument("--baseline-out", default="data/sweep/mi355x-baseline-configs.csv")
    ap.add_argument("--tag-prefix", default="s", help="first letter(s) of every shape tag")
    ap.add_argument("--exclude", action="append", default=[],
                    help="a registered sweep whose shapes this one must not repeat (a held-out set); repeatable")
    ap.add_argument("--note", action="append", default=[], help="an extra header line")
    ints = lambda s: tuple(int(v) for v in s.split(","))  # noqa: E731
    ap.add_argument("--mn-values", type=ints, default=MN_CHOICES, help="the M and N values, comma-separated")
    ap.add_argument("--k-values", type=ints, default=K_CHOICES, help="the K values, comma-separated")
    args = ap.parse_args(argv)
    os.makedirs(os.path.dirname(args.out) or ".", exist_ok=True)
    exclude = []
    if args.exclude:
        from ridge_amd import tables as T
        for path in args.exclude:
            exclude += [s[:3] for s in T.read_shapes(path)]
    try:
        write_registered(args.out, args.seed, args.tag_prefix, exclude, args.note, args.mn_values, args.k_values)
    except ValueError as e:
        raise SystemExit("ridge_amd.sweep: %s" % e)
    if args.baseline_out != "-":
        write_baseline(args.baseline_out)
    print("wrote", args.out, "" if args.baseline_out == "-" else "and " + args.baseline_out)


if __name__ == "__main__":
    main()
