"""CPU restatement of jinfer's CSR-grouped MoE dispatch. TEST INFRASTRUCTURE ONLY.

Follows ``jinfer/jinfer-kernels/src/main/java/com/qxotic/jinfer/kernels/Moe.java``:

* ``dispatch_csr``  -- the CSR build of ``Moe.dispatch`` (Moe.java:188-206): offsets = exclusive prefix
  sum of the per-expert counts, then a cursor per expert hands out slots to the routes in (s, k) order;
* ``gather``        -- Moe.java:214-222, ``g[slot] = x[rowByExpert[slot]]``;
* ``combine``       -- Moe.java:208 and 223-231: ``out`` zero-filled, then the experts in ascending order
  add ``prob · y`` to their rows with ``Ops.saxpyInPlace``'s fused multiply-add (Ops.java:688-725);
* ``mm_grouped``    -- the per-expert ``MatMul.gemm`` calls of the dispatch closure (GptOss.java:295-314),
  each one jam matmul of the expert's rows, through the int8 oracle (jo_mm_int8, jam's own routing);
* ``select_topk``   -- ``Moe.selectTopK`` (Moe.java:76-127: k argmax passes per row, the first maximum winning
  by strict ``>``, each winner masked to -Infinity in the selection array; combine weights from a second
  array in the two-source form; counts re-zeroed then filled), followed by one of the weight steps callers
  run on ``rowTopP``: gpt-oss's softmax over the k selected logits times ``expertWeightsScale``
  (GptOss.java:320-345) or ``Moe.normalizeTopP`` (Moe.java:146-152), and ``Moe.dispatch``'s fold of a
  per-expert ``expertScale`` into the combine weight (Moe.java:187-203).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg may import this module.
"""
from __future__ import annotations

import numpy as np


def dispatch_csr(route_expert: np.ndarray, n_experts: int):
    """(counts[E], offsets[E+1], slot_route[R], route_slot[R]) as Moe.dispatch builds them. A route whose
    expert id is outside [0, E) takes no slot (route_slot -1); slot_route entries past offsets[E] are -1."""
    re = np.asarray(route_expert, np.int64).ravel()
    counts = np.zeros(n_experts, np.int64)
    for e in re:
        if 0 <= e < n_experts:
            counts[e] += 1
    offsets = np.zeros(n_experts + 1, np.int64)
    offsets[1:] = np.cumsum(counts)
    cursor = offsets[:-1].copy()
    slot_route = np.full(len(re), -1, np.int64)
    route_slot = np.full(len(re), -1, np.int64)
    for r, e in enumerate(re):   # (s, k) order: r = s * topk + k
        if 0 <= e < n_experts:
            pos = cursor[e]
            cursor[e] += 1
            slot_route[pos] = r
            route_slot[r] = pos
    return counts, offsets, slot_route, route_slot


def gather(x: np.ndarray, slot_route: np.ndarray, total: int, topk: int) -> np.ndarray:
    return np.stack([x[slot_route[j] // topk] for j in range(total)]) if total else x[:0].copy()


def _fma32(a: np.float32, b: np.ndarray, c: np.ndarray) -> np.ndarray:
    """f32 fused multiply-add, one rounding: the product of two f32 is exact in the 64-bit mantissa of
    x86 long double and the sum is rounded once there before the final f32 rounding (exact for the
    operand ranges the tests use)."""
    r = np.longdouble(a) * b.astype(np.longdouble) + c.astype(np.longdouble)
    return r.astype(np.float32)


def combine(y: np.ndarray, route_expert: np.ndarray, route_prob: np.ndarray, route_slot: np.ndarray, seq: int,
            topk: int, n_experts: int) -> np.ndarray:
    dim = y.shape[1]
    out = np.zeros((seq, dim), np.float32)
    for e in range(n_experts):          # Moe.java:223: experts in ascending order
        for s in range(seq):            # then the expert's rows in slot order ((s, k) order)
            for k in range(topk):
                r = s * topk + k
                if route_expert[r] == e and route_slot[r] >= 0:
                    out[s] = _fma32(np.float32(route_prob[r]), y[route_slot[r]], out[s])
    return out


def mm_grouped(oracle, dt: int, w_experts: list, a: np.ndarray, counts, m: int, k: int) -> np.ndarray:
    """Per-expert jam matmuls over the CSR rows of a; rows past sum(counts) stay zero."""
    out = np.zeros((a.shape[0], m), np.float32)
    o = 0
    for e, n in enumerate(counts):
        n = int(n)
        if n > 0:
            out[o:o + n] = oracle.mm_int8(dt, w_experts[e], np.ascontiguousarray(a[o:o + n]), m, n, k)
        o += n
    return out


TOPK_RAW, TOPK_SOFTMAX, TOPK_NORMALIZE = 0, 1, 2


def select_topk(selection: np.ndarray, topk: int, weights: np.ndarray | None = None, mode: int = TOPK_RAW,
                weights_scale: float = 1.0, expert_scale: np.ndarray | None = None):
    """(route_expert[rows*topk] int, route_prob[rows*topk] f32, counts[E] int, selection after masking).
    ``selection`` [rows][E] f32 is copied, not changed; the returned copy carries the -Inf masks jinfer
    leaves in its array."""
    sel = np.array(selection, np.float32, copy=True)
    w = sel if weights is None else np.asarray(weights, np.float32)
    rows, E = sel.shape
    re = np.zeros(rows * topk, np.int64)
    rp = np.zeros(rows * topk, np.float32)
    counts = np.zeros(E, np.int64)
    for s in range(rows):
        for ki in range(topk):
            best, best_val = 0, np.float32(-np.inf)
            for e in range(E):
                v = sel[s, e]
                if v > best_val:   # NaN compares false: never taken, as in Java
                    best_val, best = v, e
            re[s * topk + ki] = best
            rp[s * topk + ki] = w[s, best]   # read before the mask (one-source form: the same array)
            sel[s, best] = np.float32(-np.inf)
            counts[best] += 1
        base = s * topk
        p = rp[base:base + topk]
        if mode == TOPK_SOFTMAX:           # GptOss.selectExperts: softmax over the raw selected logits
            mx = np.float32(-np.inf)
            for v in p:
                mx = np.float32(np.nan) if (np.isnan(mx) or np.isnan(v)) else max(mx, v)   # Math.max
            total = np.float32(0.0)
            vals = np.zeros(topk, np.float32)
            for i in range(topk):
                vals[i] = np.float32(np.exp(np.float64(np.float32(p[i] - mx))))      # (float) Math.exp(double)
                total = np.float32(total + vals[i])
            inv = np.float32(0.0) if total == 0 else np.float32(np.float32(1.0) / total)
            for i in range(topk):
                p[i] = np.float32(np.float32(vals[i] * inv) * np.float32(weights_scale))
        elif mode == TOPK_NORMALIZE:       # Moe.normalizeTopP
            total = np.float32(0.0)
            for i in range(topk):
                total = np.float32(total + p[i])
            for i in range(topk):
                p[i] = np.float32(p[i] / total)
        if expert_scale is not None:       # Moe.dispatch: probByExpert = rowTopP * expertScale[e]
            for i in range(topk):
                p[i] = np.float32(p[i] * np.float32(expert_scale[re[base + i]]))
        rp[base:base + topk] = p
    return re, rp, counts, sel
