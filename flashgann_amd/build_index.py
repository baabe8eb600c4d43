"""Command-line codebook and ground-truth builder for the reference's inputs.

The reference consumes a prebuilt SymphonyQG-style codebook and an .ivecs
ground truth (main.cu:57-59, include/qg.hpp:17-42) and ships no tool that
makes either (README.md:12).  This module writes both from .fvecs files:

  python -m flashgann_amd.build_index index base.fvecs out.index [--degree 32]
         [--metric auto|l2|ip] [--device cuda|cpu] [--seed 1]
  python -m flashgann_amd.build_index gt base.fvecs query.fvecs out.ivecs
         [--k 100] [--metric auto|l2|ip] [--device cuda|cpu]

`--metric auto` follows the reference's rule (include/metric.hpp:13-28): inner
product when the base path contains "text2image1m", L2 otherwise.  The
codebook's sign vector is drawn from the seeded generator of `datasets`.
"""
from __future__ import annotations

import argparse
import sys
import time

import numpy as np


def _metric(name: str, base_path: str) -> bool:
    """True for inner product."""
    if name == "auto":
        return "text2image1m" in base_path.lower()
    return name == "ip"


def _device(name: str) -> str:
    if name == "cuda":
        import torch
        if not torch.cuda.is_available():
            raise SystemExit("--device cuda: no GPU is visible")
    return name


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(prog="python -m flashgann_amd.build_index", description=__doc__.splitlines()[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    pi = sub.add_parser("index", help="build a codebook in the reference's layout")
    pi.add_argument("base")
    pi.add_argument("out")
    pi.add_argument("--degree", type=int, default=32)
    pi.add_argument("--seed", type=int, default=1, help="seed of the rotation's sign vector")
    pg = sub.add_parser("gt", help="exact top-k ground truth as .ivecs")
    pg.add_argument("base")
    pg.add_argument("queries")
    pg.add_argument("out")
    pg.add_argument("--k", type=int, default=100)
    for p in (pi, pg):
        p.add_argument("--metric", choices=("auto", "l2", "ip"), default="auto")
        p.add_argument("--device", choices=("cuda", "cpu"), default="cuda")
    args = ap.parse_args(argv)

    from . import builder, datasets
    from .codebook import padded_dim_for, read_fvecs, write_ivecs

    use_ip = _metric(args.metric, args.base)
    dev = _device(args.device)
    base = read_fvecs(args.base)
    t0 = time.time()
    if args.cmd == "index":
        signs = datasets.signs_for(padded_dim_for(base.shape[1]), args.seed)
        cb = builder.build_codebook(base, args.degree, signs, use_ip=use_ip, device=dev)
        cb.save(args.out)
        print(f"codebook: {base.shape[0]} nodes, dim {base.shape[1]}, degree {args.degree}, "
              f"{'ip' if use_ip else 'l2'}, entry {cb.entry} -> {args.out} ({time.time() - t0:.1f} s)")
    else:
        q = read_fvecs(args.queries)
        if q.shape[1] != base.shape[1]:
            raise SystemExit(f"query dimension {q.shape[1]} does not match base dimension {base.shape[1]}")
        gt = builder.ground_truth(base, q, args.k, device=dev, use_ip=use_ip)
        write_ivecs(args.out, np.ascontiguousarray(gt, dtype=np.int32))
        print(f"ground truth: {q.shape[0]} queries, top {args.k}, {'ip' if use_ip else 'l2'} -> {args.out} "
              f"({time.time() - t0:.1f} s)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
