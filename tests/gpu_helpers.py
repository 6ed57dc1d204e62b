"""Shared helpers for the GPU parity tests (comparison rules of the parity bar)."""

import numpy as np

REL_L2_BAR = 1e-3       # layer outputs, fp32-accumulated BF16/MX paths
TIE_GAP = 1e-6          # top-k may differ only between experts whose scores differ by less


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))


def ids_match(gpu_ids, ref_ids, ref_scores) -> bool:
    """Top-k ids identical except where adjacent reference scores differ by < TIE_GAP.

    ``ref_scores[t]`` are the per-expert values the reference ranks by (router logits for
    softmax; sigmoid(logit) + bias for noaux_tc; sqrt(softplus(logit)) + bias for
    sqrt-softplus)."""
    gpu_ids = np.asarray(gpu_ids)
    ref_ids = np.asarray(ref_ids)
    for t in range(ref_ids.shape[0]):
        g, r = list(gpu_ids[t]), list(ref_ids[t])
        if g == r:
            continue
        s = np.asarray(ref_scores[t], np.float64)
        for a, b in zip(g, r):
            if a != b and abs(s[a] - s[b]) >= TIE_GAP:
                return False
    return True


def noaux_scores(logits, bias):
    logits = np.asarray(logits, np.float64)
    g = 1.0 / (1.0 + np.exp(-logits))
    return g + (0.0 if bias is None else np.asarray(bias, np.float64)[None, :])


def sqrt_softplus_scores(logits, bias):
    g = np.sqrt(np.logaddexp(0.0, np.asarray(logits, np.float64)))
    return g + (0.0 if bias is None else np.asarray(bias, np.float64)[None, :])
