"""CPU oracle of the FLAT-ATTENTION hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import this package, and only as the checker or as the timed CPU baseline. The product
library (``flat-attention_amd``) never imports, links or calls it.

This module is a thin numpy/ctypes wrapper over ``liboracle.so`` (built from ``oracle.c``
by ``oracle/Makefile``), which restates the reference crate's scalar Rust oracles
(``src/lib.rs:454``, ``src/grouped.rs:81``, ``src/rotary_grouped.rs:57``,
``src/projection_asymmetric.rs:97``, ``src/chunked_projection_prefill.rs:63``,
``src/backward_grouped.rs:17``) loop for
loop. Each wrapper returns ``(out, lse)`` float32 arrays or raises ``OracleError``.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_U64 = ctypes.c_uint64
_F = ctypes.c_float
_I = ctypes.c_int
_P = ctypes.c_void_p
UNIT_ALL = (0, 2**64 - 1)


class OracleError(RuntimeError):
    def __init__(self, code: int, what: str):
        super().__init__(f"oracle {what} failed with status {code}")
        self.code = code


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(_P)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _check(rc, what):
    if rc != 0:
        raise OracleError(rc, what)


def resolved_scale(head_dim: int, scale: float | None = None) -> float:
    out = _F()
    rc = lib().ora_resolved_scale(_I(scale is not None), _F(scale or 0.0), _U64(head_dim),
                                  ctypes.byref(out))
    _check(rc, "resolved_scale")
    return out.value


def forward(q, k, v, batch, heads, seq, dim, causal, scale=None, units=UNIT_ALL, threads=1):
    """forward_reference src/lib.rs:454 on [B,H,S,D] f32."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    s = resolved_scale(dim, scale)
    out = np.zeros(batch * heads * seq * dim, np.float32)
    lse = np.zeros(batch * heads * seq, np.float32)
    rc = lib().ora_forward(_ptr(q), _ptr(k), _ptr(v), _U64(batch), _U64(heads), _U64(seq),
                           _U64(dim), _I(int(causal)), _F(s), _ptr(out), _ptr(lse),
                           _U64(units[0]), _U64(units[1]), _I(threads))
    _check(rc, "forward")
    return out, lse


def forward_grouped(q, k, v, batch, q_heads, kv_heads, seq, dim, causal, scale=None,
                    units=UNIT_ALL, threads=1):
    """forward_reference_grouped src/grouped.rs:81."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    s = resolved_scale(dim, scale)
    out = np.zeros(batch * q_heads * seq * dim, np.float32)
    lse = np.zeros(batch * q_heads * seq, np.float32)
    rc = lib().ora_forward_grouped(_ptr(q), _ptr(k), _ptr(v), _U64(batch), _U64(q_heads),
                                   _U64(kv_heads), _U64(seq), _U64(dim), _I(int(causal)),
                                   _F(s), _ptr(out), _ptr(lse), _U64(units[0]), _U64(units[1]),
                                   _I(threads))
    _check(rc, "forward_grouped")
    return out, lse


def backward_grouped(q, k, v, d_out, out, lse, batch, q_heads, kv_heads, seq, dim, causal,
                     scale=None, threads=1):
    """backward_reference_grouped src/backward_grouped.rs:17 -> (dq, dk, dv) float32."""
    q, k, v, d_out, out, lse = (_f32(x) for x in (q, k, v, d_out, out, lse))
    s = resolved_scale(dim, scale)
    qn, kvn = batch * q_heads * seq * dim, batch * kv_heads * seq * dim
    dq = np.zeros(qn, np.float32)
    dk = np.zeros(kvn, np.float32)
    dv = np.zeros(kvn, np.float32)
    rc = lib().ora_backward_grouped(_ptr(q), _ptr(k), _ptr(v), _ptr(d_out), _ptr(out), _ptr(lse),
                                    _U64(batch), _U64(q_heads), _U64(kv_heads), _U64(seq),
                                    _U64(dim), _I(int(causal)), _F(s), _ptr(dq), _ptr(dk),
                                    _ptr(dv), _I(threads))
    _check(rc, "backward_grouped")
    return dq, dk, dv


def forward_grouped_rope(q, k, v, batch, q_heads, kv_heads, seq, dim, causal, theta,
                         position_offset=0, scale=None, units=UNIT_ALL, threads=1):
    """forward_reference_grouped_rope src/rotary_grouped.rs:57."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    s = resolved_scale(dim, scale)
    out = np.zeros(batch * q_heads * seq * dim, np.float32)
    lse = np.zeros(batch * q_heads * seq, np.float32)
    rc = lib().ora_forward_grouped_rope(_ptr(q), _ptr(k), _ptr(v), _U64(batch), _U64(q_heads),
                                        _U64(kv_heads), _U64(seq), _U64(dim), _I(int(causal)),
                                        _F(s), _F(theta), _U64(position_offset), _ptr(out),
                                        _ptr(lse), _U64(units[0]), _U64(units[1]), _I(threads))
    _check(rc, "forward_grouped_rope")
    return out, lse


def forward_projection_asymmetric(q, k, v, batch, q_heads, kv_heads, query_len, kv_len, dim,
                                  query_position_offset, causal, theta=None, q_rope_offset=0,
                                  kv_rope_offset=0, rotate_k=True, scale=None, units=UNIT_ALL,
                                  threads=1):
    """forward_reference_projection_grouped_rope_asymmetric src/projection_asymmetric.rs:97.

    ``theta=None`` disables RoPE; ``rotate_k=False`` treats K as pre-rotated."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    s = resolved_scale(dim, scale)
    out = np.zeros(batch * query_len * q_heads * dim, np.float32)
    lse = np.zeros(batch * q_heads * query_len, np.float32)
    rc = lib().ora_forward_projection_asymmetric(
        _ptr(q), _ptr(k), _ptr(v), _U64(batch), _U64(q_heads), _U64(kv_heads), _U64(query_len),
        _U64(kv_len), _U64(dim), _U64(query_position_offset), _I(int(causal)), _F(s),
        _I(theta is not None), _F(theta or 0.0), _U64(q_rope_offset), _U64(kv_rope_offset),
        _I(int(rotate_k)), _ptr(out), _ptr(lse), _U64(units[0]), _U64(units[1]), _I(threads))
    _check(rc, "forward_projection_asymmetric")
    return out, lse


def chunked_prefill(q, k, v, batch, q_heads, kv_heads, seq, dim, causal, theta,
                    position_offset, chunk, scale=None):
    """forward_reference_projection_grouped_rope_chunked_prefill
    src/chunked_projection_prefill.rs:63."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    s = resolved_scale(dim, scale)
    out = np.zeros(batch * seq * q_heads * dim, np.float32)
    lse = np.zeros(batch * q_heads * seq, np.float32)
    rc = lib().ora_chunked_prefill(_ptr(q), _ptr(k), _ptr(v), _U64(batch), _U64(q_heads),
                                   _U64(kv_heads), _U64(seq), _U64(dim), _I(int(causal)),
                                   _F(s), _F(theta), _U64(position_offset), _U64(chunk),
                                   _ptr(out), _ptr(lse))
    _check(rc, "chunked_prefill")
    return out, lse


def rope_rotate_rows(x, rows, heads, dim, theta, position_offset=0, positions=None):
    """Materialise RoPE on a [rows, heads*dim] tensor (rotated_pair src/rotary_grouped.rs:37)."""
    x = _f32(x)
    out = np.empty_like(x)
    pos = None if positions is None else np.ascontiguousarray(positions, dtype=np.int64)
    rc = lib().ora_rope_rotate_rows(_ptr(x), _ptr(out), _U64(rows), _U64(heads), _U64(dim),
                                    _F(theta), _U64(position_offset), _ptr(pos))
    _check(rc, "rope_rotate_rows")
    return out


def paged_decode(q, k_pool, v_pool, physical_pages, page_size, block_tables, ctx_lens,
                 q_heads, kv_heads, dim, causal, theta, q_positions=None, scale=None,
                 seqs=UNIT_ALL, threads=1):
    """Paged q_len=1 decode: gather by block table, then the asymmetric oracle with
    pre-rotated K (tests/m16_paged_decode.rs:171)."""
    q, kp, vp = _f32(q), _f32(k_pool), _f32(v_pool)
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    cl = np.ascontiguousarray(ctx_lens, dtype=np.int32)
    qp = None if q_positions is None else np.ascontiguousarray(q_positions, dtype=np.int32)
    n = cl.shape[0]
    s = resolved_scale(dim, scale)
    out = np.zeros(n * q_heads * dim, np.float32)
    lse = np.zeros(n * q_heads, np.float32)
    rc = lib().ora_paged_decode(_ptr(q), _ptr(kp), _ptr(vp), _U64(physical_pages),
                                _U64(page_size), _ptr(bt), _U64(bt.shape[1]), _ptr(cl), _ptr(qp),
                                _U64(n), _U64(q_heads), _U64(kv_heads), _U64(dim),
                                _I(int(causal)), _F(s), _F(theta), _ptr(out), _ptr(lse),
                                _U64(seqs[0]), _U64(seqs[1]), _I(threads))
    _check(rc, "paged_decode")
    return out, lse


def paged_prefill(q, k_pool, v_pool, physical_pages, page_size, block_tables, q_heads,
                  kv_heads, query_len, kv_len, dim, query_position_offset, causal, theta,
                  q_rope_offset, scale=None, seqs=UNIT_ALL, threads=1):
    """Chunked prefill over the page pool (pre-rotated K), per-sequence asymmetric oracle."""
    q, kp, vp = _f32(q), _f32(k_pool), _f32(v_pool)
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    n = bt.shape[0]
    s = resolved_scale(dim, scale)
    out = np.zeros(n * query_len * q_heads * dim, np.float32)
    lse = np.zeros(n * q_heads * query_len, np.float32)
    rc = lib().ora_paged_prefill(_ptr(q), _ptr(kp), _ptr(vp), _U64(physical_pages),
                                 _U64(page_size), _ptr(bt), _U64(bt.shape[1]), _U64(n),
                                 _U64(q_heads), _U64(kv_heads), _U64(query_len), _U64(kv_len),
                                 _U64(dim), _U64(query_position_offset), _I(int(causal)), _F(s),
                                 _F(theta), _U64(q_rope_offset), _ptr(out), _ptr(lse),
                                 _U64(seqs[0]), _U64(seqs[1]), _I(threads))
    _check(rc, "paged_prefill")
    return out, lse


def f32_to_bf16(x):
    x = _f32(x)
    out = np.empty(x.shape, np.uint16)
    lib().ora_f32_to_bf16_array(_ptr(x), _ptr(out), _U64(x.size))
    return out


def bf16_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().ora_bf16_to_f32_array(_ptr(h), _ptr(out), _U64(h.size))
    return out


def f32_to_f16(x):
    x = _f32(x)
    out = np.empty(x.shape, np.uint16)
    lib().ora_f32_to_f16_array(_ptr(x), _ptr(out), _U64(x.size))
    return out


def f16_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().ora_f16_to_f32_array(_ptr(h), _ptr(out), _U64(h.size))
    return out


def fill_normal(n: int, seed: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().ora_fill_normal(_ptr(out), _U64(n), _U64(seed))
    return out
