"""Oracle: adaptive-format decode attention (test infrastructure).

Restates the reference's Triton kernel
(triton_adaptive_format_attention.py:92-225) in float64: for each (batch,
head) row, over the max_selected_pages entries of page_ids,
  * id < 0, or format SKIP (3): no contribution;
  * SPARSE (2): no contribution (score -inf, :211);
  * FP16 (0): K, V rows as stored;
  * INT8 (1): K = code * k_scale, V = code * v_scale (float32 products);
  * any other format: page_size zero K and V rows, score 0 (the masked loads
    return 0 and the score is kept, :200-211);
softmax with scale 1/sqrt(D) over all contributing tokens; a row with no
contribution outputs zeros (:217-218). This build skips ids >= num_pages
(the reference reads out of bounds there).

Pinned by: on FP16 / INT8 / SKIP / SPARSE pages with -1 holes it equals
oracle.decode.paged_decode_oracle (pinned by golden vectors and brute force)
with SPARSE mapped to SKIP and the holes dropped; closed forms for the
zero-row format, an all-SKIP row and an empty row (tests/test_oracle_adaptive.py).
"""
from __future__ import annotations

import math

import numpy as np


def adaptive_decode_oracle(q, page_ids, page_formats, k16, v16, k8=None, v8=None, ks=None, vs=None):
    q = np.asarray(q, np.float64)
    B, H, D = q.shape
    NP, PS = k16.shape[0], k16.shape[1]
    out = np.zeros((B, H, D))
    for b in range(B):
        for h in range(H):
            K, V = [], []
            for pid in np.asarray(page_ids[b, h]).tolist():
                if pid < 0 or pid >= NP:
                    continue
                f = int(page_formats[pid])
                if f in (2, 3):
                    continue
                if f == 0:
                    K.append(np.asarray(k16[pid], np.float64))
                    V.append(np.asarray(v16[pid], np.float64))
                elif f == 1 and k8 is not None:
                    K.append((np.asarray(k8[pid], np.float32) * np.float32(ks[pid])).astype(np.float64))
                    V.append((np.asarray(v8[pid], np.float32) * np.float32(vs[pid])).astype(np.float64))
                else:
                    K.append(np.zeros((PS, D)))
                    V.append(np.zeros((PS, D)))
            if not K:
                continue
            Kc, Vc = np.concatenate(K), np.concatenate(V)
            s = Kc @ q[b, h] / math.sqrt(D)
            p = np.exp(s - s.max())
            out[b, h] = p @ Vc / p.sum()
    return out
