"""Port of the reference's butterquant sliding-attention parity scenario
(tests/test_sliding_attention_degree_parity.mojo), degree 1.

Shared by the CPU oracle test and the GPU parity test: deterministic
content_value inputs, three sequences on fixed 2-page rings of 64-token pages,
the reference's 10-step prefill/decode schedule, identity RoPE and unit norm
gains, and the scalar reference_head (exact exp) with tolerance 0.05.
"""
from __future__ import annotations

import math

import numpy as np

HEAD_DIM = 256
NUM_Q = 16
NUM_KV = 8
GQA = NUM_Q // NUM_KV
Q_STRIDE = NUM_Q * HEAD_DIM
KV_STRIDE = NUM_KV * HEAD_DIM
PAGE_LEN = 64
WINDOW = 64
RING_PAGES = 2
CACHE_SIZE = RING_PAGES * PAGE_LEN
ROPE_HALF = HEAD_DIM // 2
PAIR_STRIDE = HEAD_DIM // 2
SQRT_HD = np.float32(16.0)
HD_EPS = np.float32(HEAD_DIM) * np.float32(1e-6)
NUM_PAGES = 6
CACHE_ROWS = NUM_PAGES * PAGE_LEN
ROPE_ROWS = 512
POOL_WORKERS = 4  # cap
TOL = 0.05

MASK64 = (1 << 64) - 1


def sequence_pages(seq: int) -> list[int]:  # :44-55
    return {0: [3, 1], 1: [0, 4]}.get(seq, [2, 5])


def content_value(key: np.ndarray, column: np.ndarray, salt: int) -> np.ndarray:
    """content_value (:58-65), vectorised over uint64 with wraparound."""
    key = np.asarray(key, dtype=np.uint64)
    column = np.asarray(column, dtype=np.uint64)
    with np.errstate(over="ignore"):
        h = (key * np.uint64(2654435761) + column * np.uint64(2246822519)
             + np.uint64(salt) * np.uint64(3266489917))
        h ^= h >> np.uint64(13)
        h *= np.uint64(1099511628211)
        h ^= h >> np.uint64(29)
    v = (h % np.uint64(17)).astype(np.int64) - 8
    return v.astype(np.float32) * np.float32(0.05)


def to_bf16_bits(f: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + ((u >> 16) & 1) + 0x7FFF) >> 16).astype(np.uint16)


def schedule() -> list[list[tuple[int, int, int]]]:
    """(seq, start, count) runs per step (:366-413)."""
    return [
        [(0, 0, 64)],
        [(0, 64, 64)],
        [(0, 128, 22), (1, 0, 42)],
        [(1, 42, 64)],
        [(1, 106, 14), (2, 0, 50)],
        [(2, 50, 64)],
        [(2, 114, 64)],
        [(0, 150, 1), (1, 120, 1), (2, 178, 22)],
        [(0, 151, 1), (1, 121, 1), (2, 200, 1)],
        [(0, 152, 1)],
    ]


def step_inputs(runs_spec):
    """Token lists, q/k/v bf16 sources and the run table for one step."""
    tok_seq, tok_pos, runs, rows = [], [], [], []
    for seq, start, count in runs_spec:
        runs.append([len(tok_seq), start, len(rows), RING_PAGES])
        rows.extend(p * PAGE_LEN for p in sequence_pages(seq))
        for p in range(start, start + count):
            tok_seq.append(seq)
            tok_pos.append(p)
    n = len(tok_seq)
    key = np.asarray(tok_seq, dtype=np.uint64) * np.uint64(512) + np.asarray(tok_pos, dtype=np.uint64)
    qc = np.arange(Q_STRIDE, dtype=np.uint64)
    kc = np.arange(KV_STRIDE, dtype=np.uint64)
    q = to_bf16_bits(content_value(key[:, None], qc[None, :], 1)).reshape(-1)
    k = to_bf16_bits(content_value(key[:, None], kc[None, :], 2)).reshape(-1)
    v = to_bf16_bits(content_value(key[:, None], kc[None, :], 3)).reshape(-1)
    return (tok_seq, tok_pos, np.asarray(runs, dtype=np.int32),
            np.asarray(rows, dtype=np.int32), q, k, v, n)


def constant_tables():
    cos = np.ones(ROPE_ROWS * ROPE_HALF, dtype=np.float32)
    sin = np.zeros(ROPE_ROWS * ROPE_HALF, dtype=np.float32)
    norm = to_bf16_bits(np.ones(HEAD_DIM, dtype=np.float32))
    return cos, sin, norm


def ring_slot(pos: int, pages: list[int]) -> int:  # :83-86
    return pages[(pos // PAGE_LEN) % RING_PAGES] * PAGE_LEN + pos % PAGE_LEN


def reference_head(head, pos, k_cache, k_scale, v_cache, v_scale, pages, q_row, qf):
    """reference_head (:89-141) at degree 1: exact exp, sequential online
    softmax over the window, f32 state."""
    local_kv = head // GQA
    inv127 = np.float32(1.0) / np.float32(127.0)
    inv127sq = inv127 * inv127
    m = np.float32(-1e30)
    l = np.float32(0.0)
    acc = np.zeros(HEAD_DIM, dtype=np.float32)
    lo = max(0, pos - WINDOW + 1)
    q = q_row.astype(np.int64)
    for p in range(lo, pos + 1):
        slot = ring_slot(p, pages)
        kh = k_cache[slot * KV_STRIDE + local_kv * HEAD_DIM:][:HEAD_DIM].astype(np.int64)
        dot = int(np.dot(kh, q))
        ks = k_scale[slot * NUM_KV + local_kv]
        s = np.float32(np.float32(np.float32(np.float32(dot) * qf) * ks) * inv127sq)
        m_new = s if s > m else m
        corr = np.float32(math.exp(float(m - m_new)))
        w = np.float32(math.exp(float(s - m_new)))
        l = np.float32(l * corr + w)
        vs = v_scale[slot * NUM_KV + local_kv]
        vh = v_cache[slot * KV_STRIDE + local_kv * HEAD_DIM:][:HEAD_DIM].astype(np.float32)
        vw = np.float32(np.float32(w * vs) * inv127)
        acc = (acc * corr + vh * vw).astype(np.float32)
        m = m_new
    if l > 0:
        acc = acc * (np.float32(1.0) / l)
    return acc


def check_step(tok_seq, tok_pos, runs_spec, q_i8, f_q, k_cache, k_scale, v_cache, v_scale,
               out_bits) -> float:
    """Worst |out - reference_head| over the step's tokens and heads."""
    out = (out_bits.astype(np.uint32) << 16).view(np.float32).reshape(-1, NUM_Q, HEAD_DIM)
    worst = 0.0
    for t in range(len(tok_seq)):
        pages = sequence_pages(tok_seq[t])
        for h in range(NUM_Q):
            ref = reference_head(h, tok_pos[t], k_cache, k_scale, v_cache, v_scale, pages,
                                 q_i8[t * Q_STRIDE + h * HEAD_DIM:][:HEAD_DIM],
                                 f_q[t * NUM_Q + h])
            worst = max(worst, float(np.max(np.abs(out[t, h] - ref))))
    return worst
