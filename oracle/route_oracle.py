"""CPU restatement of the MoE router's routing step (vllm_sm80/kernels/moe/
route.py:333-355 keys, :426-571 selection and weights; the sigmoid/bias form
of its docstring, route.py:1-40) and of softmax routing.

TEST INFRASTRUCTURE ONLY.  Only tests/ may import this module, as the
checker; the product path (vllm-cmp170hx_amd/) never does.

Selection is a function of the logits; the device computes its own FP32
logits (one fixed summation order), so the tests pin the logits against an
FP64 product separately and feed the device's logits to ``route``.  Scores
are FP32 NumPy (tanh / exp); the device's FP32 tanhf / expf may differ from
NumPy's by an ulp, so ``route`` also returns each row's key gaps for the
tests' near-tie allowance.  Pinned by: ties going to the lower expert on
hand-made rows, weights summing to `scale` after renormalization, and the
softmax keys' order equal to the logits' order (tests/test_oracle_route.py).
"""

from __future__ import annotations

import numpy as np


def logits_fp64(x_f32: np.ndarray, w_f32: np.ndarray) -> np.ndarray:
    """x [M, K] and W [E, K] (exact bf16 / fp16 values) -> x W^T in FP64."""
    return x_f32.astype(np.float64) @ w_f32.astype(np.float64).T


def scores(logits: np.ndarray, sigmoid: bool) -> np.ndarray:
    l = logits.astype(np.float32)
    if sigmoid:
        return (np.float32(0.5) * np.tanh(np.float32(0.5) * l) + np.float32(0.5)).astype(np.float32)
    e = np.exp(l - l.max(axis=1, keepdims=True)).astype(np.float32)
    return (e / e.sum(axis=1, keepdims=True, dtype=np.float32)).astype(np.float32)


def route(logits, topk, sigmoid=True, bias=None, renormalize=True, scale=1.0):
    """-> (ids [M, topk] int32, weights [M, topk] float32, gaps [M]): the top-k
    by key (ties to the lower expert), weights = selected scores, divided by
    (sum + 1e-20) if renormalize, times scale; gaps = the smallest key
    difference between the k-th chosen and the best unchosen expert."""
    s = scores(logits, sigmoid)
    key = s + bias.astype(np.float32)[None, :] if sigmoid else s
    M, E = key.shape
    ids = np.zeros((M, topk), np.int32)
    w = np.zeros((M, topk), np.float32)
    gaps = np.zeros(M, np.float64)
    for m in range(M):
        order = sorted(range(E), key=lambda e: (-float(key[m, e]), e))
        ids[m] = order[:topk]
        sel = s[m, ids[m]].astype(np.float32)
        tot = np.float32(0.0)
        for v in sel:
            tot = np.float32(tot + v)
        ww = sel / np.float32(tot + np.float32(1e-20)) if renormalize else sel
        w[m] = (ww * np.float32(scale)).astype(np.float32)
        gaps[m] = float(key[m, order[topk - 1]]) - float(key[m, order[topk]]) if topk < E else np.inf
    return ids, w, gaps
