"""Selection rules of the path, restated on the CPU (test infrastructure only).

* ``radix_key``: the order-preserving u32 key of an f32 (glm53/check.py:94-97,
  glm53/gfx950/kernel.py:2698-2699).
* ``exact_topk``: top-k by (key descending, position ascending), the reference's
  definition of its exact top-2048 (glm53/check.py:100-117).
* ``radix_select``: the same selection computed the way the device does it, with
  MSB-first 8-bit digit histograms (deepseek_v4/gfx950/kernels/stages/indexer.py:604-802,
  glm53/gfx950/kernel.py:3000-3636). It is a second, independent implementation used
  to pin ``exact_topk`` and to restate the device algorithm.
* ``router_top8``: the sigmoid router's top-8 with lowest-id ties and the 2.5-scaled
  renormalised weights (glm53/gfx950/kernel.py:1575-1629, glm53/check.py:149-168).
* ``softmax_topk``: the MXFP4 MoE's softmax router: top-k of the logits with
  lowest-id ties, weights renormalised over the k picks.
"""

from __future__ import annotations

import numpy as np
import torch

ROUTE_SCALE = 2.5  # glm53/check.py:37 (TOP_K, ROUTE_SCALE = 8, 2.5)


def radix_key(x) -> np.ndarray:
    """float32 values (tensor or array) -> uint32 keys, larger key = larger value;
    +0 ranks above -0 (glm53/check.py:94-97)."""
    if isinstance(x, torch.Tensor):
        x = x.float().contiguous().numpy()
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.int32).astype(np.int64)
    k = np.where(b >= 0, b + (1 << 31), (~b) & 0xFFFFFFFF)
    return k.astype(np.uint32)


def exact_topk(scores, k: int) -> np.ndarray:
    """Positions of the top ``k`` of ``scores`` [n] by (key desc, position asc),
    returned in ascending position order. n <= k selects every position
    (glm53/check.py:108-113: ``torch.sort(keys, descending=True, stable=True)``)."""
    keys = radix_key(scores)
    n = keys.shape[0]
    if n <= k:
        return np.arange(n, dtype=np.int64)
    # stable argsort on the negated order keeps ascending positions among equal keys
    order = np.argsort(-keys.astype(np.int64), kind="stable")
    return np.sort(order[:k])


def radix_select(scores, k: int) -> np.ndarray:
    """``exact_topk`` computed by 8-bit MSB-first digit histograms: find the k-th
    largest key digit by digit, take every key above it and the lowest-position
    keys equal to it (indexer.py:693-781: 'compaction in ascending index, lowest-index
    ties')."""
    keys = radix_key(scores)
    n = keys.shape[0]
    if n <= k:
        return np.arange(n, dtype=np.int64)
    prefix, mask = 0, 0
    need = k  # how many of the keys matching the prefix still belong to the top-k
    for shift in (24, 16, 8, 0):
        live = (keys & np.uint32(mask)) == np.uint32(prefix)
        digit = (keys[live] >> np.uint32(shift)) & np.uint32(0xFF)
        hist = np.bincount(digit.astype(np.int64), minlength=256)
        # walk digits from 255 down until the running count reaches ``need``
        above = 0
        for d in range(255, -1, -1):
            if above + hist[d] >= need:
                break
            above += hist[d]
        need -= above
        prefix |= d << shift
        mask |= 0xFF << shift
    thresh = np.uint32(prefix)
    gt = np.nonzero(keys > thresh)[0]
    eq = np.nonzero(keys == thresh)[0][:need]
    return np.sort(np.concatenate([gt, eq]))


def router_top8(scores: torch.Tensor, bias: torch.Tensor, k: int = 8, scale: float = ROUTE_SCALE):
    """Sigmoid router selection of one or more rows.

    ``scores`` [S, E] f32 sigmoid scores, ``bias`` [E] f32. Selects by the f32 bits of
    (score + bias) descending, lowest expert id among exactly equal keys
    (glm53/gfx950/kernel.py:1575-1629); weight = score / sum of the k scores * 2.5
    (kernel.py:1626-1629). Returns (ids int64 [S, k] in pick order, weights f32 [S, k]).
    """
    s = scores.float()
    key_in = (s + bias.float()[None, :]).float()
    ids = []
    for row in range(s.shape[0]):
        keys = radix_key(key_in[row])
        order = np.argsort(-keys.astype(np.int64), kind="stable")[:k]
        ids.append(order)
    ids = torch.from_numpy(np.stack(ids)).long()
    raw = s.gather(1, ids)
    w = raw / raw.sum(-1, keepdim=True) * scale
    return ids, w.float()


def softmax_topk(logits: torch.Tensor, k: int = 8):
    """Softmax router of the MXFP4 MoE: top-k of the f32 logits (key descending,
    lowest id on exact ties), weights = softmax over the k picked logits, i.e. the
    full softmax renormalised over the picks. Returns (ids [S, k], weights [S, k])."""
    lg = logits.float()
    ids = []
    for row in range(lg.shape[0]):
        keys = radix_key(lg[row])
        ids.append(np.argsort(-keys.astype(np.int64), kind="stable")[:k])
    ids = torch.from_numpy(np.stack(ids)).long()
    picked = lg.gather(1, ids)
    w = torch.softmax(picked.double(), -1).float()
    return ids, w
