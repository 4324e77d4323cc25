"""CPU restatement of jinfer's CSR-grouped MoE dispatch. TEST INFRASTRUCTURE ONLY.

Follows ``jinfer/jinfer-kernels/src/main/java/com/qxotic/jinfer/kernels/Moe.java``:

* ``dispatch_csr``  -- the CSR build of ``Moe.dispatch`` (Moe.java:188-206): offsets = exclusive prefix
  sum of the per-expert counts, then a cursor per expert hands out slots to the routes in (s, k) order;
* ``gather``        -- Moe.java:214-222, ``g[slot] = x[rowByExpert[slot]]``;
* ``combine``       -- Moe.java:208 and 223-231: ``out`` zero-filled, then the experts in ascending order
  add ``prob · y`` to their rows with ``Ops.saxpyInPlace``'s fused multiply-add (Ops.java:688-725);
* ``mm_grouped``    -- the per-expert ``MatMul.gemm`` calls of the dispatch closure (GptOss.java:295-314),
  each one jam matmul of the expert's rows, through the int8 oracle (jo_mm_int8, jam's own routing).

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
