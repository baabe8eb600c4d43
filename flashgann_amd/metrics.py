"""Recall and the CSV run record (include/common.hpp:19-24, 49-94)."""
from __future__ import annotations

import os

import numpy as np


def compute_recall(predicted: np.ndarray, groundtruth: np.ndarray, topk: int) -> float:
    """Fraction of predicted ids found among the first min(topk, gt_k) ground
    truth ids of their query; a repeated prediction counts each time it
    appears (include/common.hpp:49-66).  Returned in float32 precision."""
    pred = np.asarray(predicted).reshape(-1, topk).astype(np.int64)
    gt = np.asarray(groundtruth)
    eval_k = min(topk, gt.shape[1])
    hits = 0
    for i in range(pred.shape[0]):
        g = gt[i, :eval_k].astype(np.int64)
        hits += int(np.isin(pred[i], g).sum())
    return float(np.float32(hits) / np.float32(pred.shape[0] * topk))


def append_run_stats_to_csv(path: str, k: int, beam: int, runtime: float, latency: float,
                            throughput: float, recall: float) -> None:
    """One row of TopK,Beam_size,Runtime,Latency,Throughput,Recall; the header
    is written when the file does not exist yet (include/common.hpp:68-94)."""
    new = not os.path.exists(path)
    with open(path, "a") as f:
        if new:
            f.write("TopK,Beam_size,Runtime,Latency,Throughput,Recall\n")
        f.write(f"{k},{beam},{runtime:.6g},{latency:.6g},{throughput:.6g},{recall:.6g}\n")
