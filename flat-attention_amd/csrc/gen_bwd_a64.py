#!/usr/bin/env python3
"""Generator of the gfx950 assembly kernel fa_bwd_dkdv_a64_bf16: dK and dV of the recompute
backward of grouped attention (bf16 storage, head_dim 128, sequence a multiple of 128, dS stored
for the dQ pass), the role of bwd_dkdv<bf16, 128, true, true> (backward.hip) with the
registers allocated by hand.

Usage: gen_bwd_a64.py OUT.s OUT_ARGS.h

Math (backward_reference_grouped src/backward_grouped.rs:17-95): per (query, key) pair of a
query head of the KV head's group, P = exp2(S * scale * log2 e - LSE * log2 e)
= exp2(scale * log2 e * (S - LSE / scale)),
dS = P (dP - delta), dV += P^T dO, dK += dS^T Q (dK takes the softmax scale at the end).

Layout. One workgroup = 4 waves = 128 keys of one (batch, kv head), 32 per wave. Each lane owns
key c = lane & 31 of its wave; K and V of that key (as stored) are the B operands of S = Q K^T
and dP = dO V^T and stay in registers. Tiles of 128 query rows of Q, dO and the per-row biases
(-LSE / scale, -delta) are moved by buffer->LDS
transfers into two LDS stages (rows of 256 bytes, 16-byte chunks XOR-swizzled, conflict-free
for both the row reads of the S/dP A operands and the transposing reads of the dV/dK B operands).
Per 32-query sub-block (32 MFMAs per wave):
  S' = -LSE / scale + Q K^T      (8 v_mfma_f32_32x32x16_bf16: the first accumulates onto the
  dP' = -delta + dO V^T           bias fragment, so no VALU subtracts)
  P = exp2(c2 S'), dS = P dP'     (c2 = scale log2 e; 16 v_mul_f32 + 16 v_exp_f32 + 16 v_mul_f32,
                                   packed to bf16 for the MFMAs)
  dV += P^T dO, dK += dS^T Q      (8 + 8 MFMAs, accumulators in 128 AGPRs)
and dS goes to the workspace the dQ pass reads (the layout of BackwardArgs::ds). The MFMAs of
S and dP of sub-block i+1 run under the softmax of sub-block i; then its dV/dK MFMAs. The next
tile's transfers are spread over the first half of the tile's MFMAs.

Tile order: query tiles outer, the group's heads inner; the first half of the key blocks sweeps
the query tiles last-first, the second half first-last from its diagonal (the workgroups of one
(batch, kv head) that run at the same time then read the same tile).

Memory safety: every global access is a buffer instruction whose resource is bounded to the
slice it may touch (8 KiB of K/V rows, a 32 KiB Q/dO tile or nothing past the last tile, the
bias rows, the dS workspace from the group on, 8 KiB of dK/dV rows); every wave runs the same
number of tiles, so every barrier is met by all four.
"""
from __future__ import annotations

import importlib.util
import os
import sys

_HERE = os.path.dirname(os.path.abspath(__file__))
_spec = importlib.util.spec_from_file_location("gen_prefill_a64",
                                               os.path.join(_HERE, "gen_prefill_a64.py"))
P = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(P)
I, Gen, fdiv = P.I, P.Gen, P.fdiv

KERNEL_BF16 = "fa_bwd_dkdv_a64_bf16"
KERNEL_F16 = "fa_bwd_dkdv_a64_f16"   # f16 storage: f16 MFMAs and conversions, else identical
KERNEL = KERNEL_BF16
F16 = False


def MF() -> str:
    return "v_mfma_f32_32x32x16_f16" if F16 else "v_mfma_f32_32x32x16_bf16"


def CVT() -> str:
    return "v_cvt_pk_f16_f32" if F16 else "v_cvt_pk_bf16_f32"

# --------------------------------------------------------------------------- kernel arguments
ARGS = [
    ("q", 0, 8), ("k", 8, 8), ("v", 16, 8), ("dout", 24, 8), ("dk", 32, 8), ("dv", 40, 8),
    ("ld", 48, 8),           # -LSE / scale of every query row, then -delta of every row (f32)
    ("ds", 56, 8),
    ("seq", 64, 4), ("group", 68, 4), ("q_heads", 72, 4), ("kv_heads", 76, 4),
    ("causal", 80, 4), ("c2", 84, 4), ("scale", 88, 4), ("ds_nb", 92, 4), ("ds_gph", 96, 4),
    ("ds_bytes", 100, 4), ("nbk", 104, 4), ("fd_nbk_m", 108, 4), ("fd_nbk_s", 112, 4),
    ("fd_kvh_m", 116, 4), ("fd_kvh_s", 120, 4), ("rows", 124, 4),
]
ARG_BYTES = 128
ARG_SGPR0 = 8


def arg(name: str, hi: bool = False) -> str:
    for n, off, sz in ARGS:
        if n == name:
            return f"s{ARG_SGPR0 + off // 4 + (1 if hi else 0)}"
    raise KeyError(name)


# --------------------------------------------------------------------------- LDS
RB = 256                   # bytes per staged row (128 bf16)
T_DO = 128 * RB            # dO tile after the Q tile
T_LD = 2 * 128 * RB        # biases: 128 x -LSE / scale, then 128 x -delta (f32)
STAGE = T_LD + 1024
DUMMY = 2 * STAGE          # bias transfers of waves 1..3 (no bytes read) land here
LDS_BYTES = 2 * STAGE + 1024
SUB = 32 * RB              # one 32-row sub-block of a tile

# --------------------------------------------------------------------------- registers
V_TID, V_LANE = 0, 1
KF = 2        # 32: K fragments (8 k-steps x 4)
VF = 34       # 32: V fragments
SACC = [66, 82]    # S' accumulators (16 each), by sub-block parity
DACC = [98, 114]   # dP' accumulators
LB = 130      # 16: bias fragment -LSE / scale of the next S chain
DB = 146      # 16: -delta
PF = 162      # 8: P packed (A operand of dV, 2 k-steps x 4)
DF = 170      # 8: dS packed (A operand of dK; stored)
RA = 4        # A-operand ring (S/dP row reads): slots 0..3 at ARING, more at ARING_X
ARING = 178   # 4 x 4
RBN = 4       # B-operand ring (dV/dK transposing reads)
BRING = 194   # RBN x 4
RO = 210      # 8: row-read offsets (m, h)
TO = 218      # 8: transposing-read offsets (m, h)
V_LDB = 226   # bias read base
V_XOFF = 227  # transfer offset of instructions 0 and 4 (Q/dO rows)
V_LDOFF = 228  # bias transfer offset
V_DSOFF = 229  # 16 * lane (dS store)
V_TMP = 230   # 8 temps
V_EPW = 238   # epilogue: LDS write base
V_EPR = 239   # epilogue: LDS read base
V_EPG = 240   # epilogue: global offset of the lane's row chunk
ARING_X = 242  # A-ring slots 4.. (4 registers each, 64-bit aligned)
V_XOFF3 = ARING_X + 4 * max(0, RA - 4)  # 3: transfer offsets of instructions 1..3 (and 5..7)
NUM_VGPR = V_XOFF3 + 3


def xoff(k: int) -> int:
    """Per-lane offset register of transfer instructions k and k + 4."""
    return V_XOFF if k == 0 else V_XOFF3 + k - 1
A_DV = 0      # dV[mb]: a[16 mb ..]
A_DK = 64     # dK[mb]: a[64 + 16 mb ..]
NUM_AGPR = 128

# SGPRs: s[0:1] kernarg pointer, s2 workgroup id, s[8:39] arguments
S_WAVE = 40
S_KB = 41
S_B = 42
S_KVH = 43
S_K0 = 44          # first key of the wave
S_QSTART = 45
S_NQT = 46
S_HH = 47          # tile: head in the group
S_QT = 48          # tile: first query
S_J = 49           # tile index
S_NT = 50          # tiles
S_STAGE = 51       # LDS byte offset of the current tile's stage
S_CUR = 52         # offset currently added to RO / TO
S_CURL = 53        # offset currently added to V_LDB
S_RQ = 56          # [56:59] Q resource of the tile being transferred
S_RO = 60          # [60:63] dO resource
S_RL = 64          # [64:67] bias resource
S_RD = 68          # [68:71] dS store resource (current tile)
S_T0, S_T1, S_T2, S_T3 = 72, 73, 74, 75
S_MASK = 76        # [76:77] diagonal mask temp
S_QH0 = 78         # first query row of the group (rows)
S_S0 = 79          # first active sub-block of the tile
S_SOFF = 81        # store soffset temp
S_KROW = 82        # first K row of the (batch, kv head): bkv * seq
S_NHH = 84         # next tile: head, first query
S_NQ = 85
S_NRQ = 86         # next tile's Q/dO resource bytes (0 past the last tile)
S_NRL = 87         # next tile's bias resource bytes
S_XST = 88         # stage the next tile goes to
S_DQ = 89          # query step between tiles of one head: +128 or -128
S_XB = 90          # LDS destination of the wave's transfers (stage + 8 KiB * wave)
S_XBL = 91         # LDS destination of the bias transfer (wave 0: stage + T_LD, else DUMMY)
S_XNQ = 92         # resource bytes of the next tile's Q / dO (0 past the last tile)
S_XNL = 93         # and of its biases
S_XSOFF = 94       # transfer soffset of instructions 4..7 (16 rows: 4096)
NUM_SGPR = 96


def vr(b, n=1):
    return f"v{b}" if n == 1 else f"v[{b}:{b + n - 1}]"


def ar(b, n=1):
    return f"a{b}" if n == 1 else f"a[{b}:{b + n - 1}]"


def sr(b, n=1):
    return f"s{b}" if n == 1 else f"s[{b}:{b + n - 1}]"


def a_slot(j: int) -> int:
    """First register of A-ring slot j % RA."""
    x = j % RA
    return ARING + 4 * x if x < 4 else ARING_X + 4 * (x - 4)


def kidx(g, t):
    return 16 * (t >> 3) + 8 * g + (t & 7)


def arow(c):
    return (c & ~12) | ((c & 4) << 1) | ((c & 8) >> 1)


def swz(r, q):
    return q ^ (((r & 3) << 2) | ((r >> 2) & 3))


# --------------------------------------------------------------------------- helpers
def res64(dst, base_name, off_lo_sgpr, off_hi_sgpr, nrec):
    """s[dst:dst+3] = buffer resource at arg base + (off_hi:off_lo), nrec bytes."""
    return [I(f"s_add_u32 {sr(dst)}, {arg(base_name)}, {off_lo_sgpr}"),
            I(f"s_addc_u32 {sr(dst + 1)}, {arg(base_name, True)}, {off_hi_sgpr}"),
            I(f"s_and_b32 {sr(dst + 1)}, {sr(dst + 1)}, 0xffff"),
            I(f"s_mov_b32 {sr(dst + 2)}, {nrec}"),
            I(f"s_mov_b32 {sr(dst + 3)}, 0x20000")]


def rows_bytes(dst_lo, dst_hi, rows_sgpr):
    """(dst_hi:dst_lo) = rows * 256 (64-bit)."""
    return [I(f"s_lshl_b32 {dst_lo}, {rows_sgpr}, 8"),
            I(f"s_lshr_b32 {dst_hi}, {rows_sgpr}, 24")]


# --------------------------------------------------------------------------- set-up
def setup(gen: Gen):
    e = gen.emit
    T0, T1, T2, T3 = (sr(S_T0), sr(S_T1), sr(S_T2), sr(S_T3))
    e([I("s_load_dwordx16 s[8:23], s[0:1], 0x0"),
       I("s_load_dwordx16 s[24:39], s[0:1], 0x40"),
       I(f"v_and_b32 {vr(V_LANE)}, 63, {vr(V_TID)}"),
       I(f"v_readfirstlane_b32 {sr(S_WAVE)}, {vr(V_TID)}"),
       I("s_waitcnt lgkmcnt(0)"),
       I(f"s_lshr_b32 {sr(S_WAVE)}, {sr(S_WAVE)}, 6")])
    # workgroup -> key block kb = bid / nbk (heaviest first under a causal mask), (b, kvh)
    e(fdiv(sr(S_KB), "s2", arg("fd_nbk_m"), arg("fd_nbk_s"), T3))
    e([I(f"s_mul_i32 {T0}, {sr(S_KB)}, {arg('nbk')}"),
       I(f"s_sub_u32 {T1}, s2, {T0}")])                                  # bkv
    e(fdiv(sr(S_B), T1, arg("fd_kvh_m"), arg("fd_kvh_s"), T3))
    e([I(f"s_mul_i32 {T0}, {sr(S_B)}, {arg('kv_heads')}"),
       I(f"s_sub_u32 {sr(S_KVH)}, {T1}, {T0}"),
       I(f"s_mul_i32 {sr(S_KROW)}, {T1}, {arg('seq')}"),                 # bkv * seq
       I(f"s_lshl_b32 {sr(S_K0)}, {sr(S_KB)}, 7"),
       I(f"s_lshl_b32 {T0}, {sr(S_WAVE)}, 5"),
       I(f"s_add_u32 {sr(S_K0)}, {sr(S_K0)}, {T0}"),                     # k0 = 128 kb + 32 w
       I(f"s_lshl_b32 {sr(S_QSTART)}, {sr(S_KB)}, 7"),
       I(f"s_cmp_eq_u32 {arg('causal')}, 0"),
       I(f"s_cselect_b32 {sr(S_QSTART)}, 0, {sr(S_QSTART)}"),
       I(f"s_sub_u32 {T0}, {arg('seq')}, {sr(S_QSTART)}"),
       I(f"s_lshr_b32 {sr(S_NQT)}, {T0}, 7"),
       I(f"s_mul_i32 {sr(S_NT)}, {sr(S_NQT)}, {arg('group')}"),
       # first query row of the group: (b * q_heads + kvh * group) * seq
       I(f"s_mul_i32 {T0}, {sr(S_B)}, {arg('q_heads')}"),
       I(f"s_mul_i32 {T1}, {sr(S_KVH)}, {arg('group')}"),
       I(f"s_add_u32 {T0}, {T0}, {T1}"),
       I(f"s_mul_i32 {sr(S_QH0)}, {T0}, {arg('seq')}")])
    # ---- K and V fragments of key k0 + c: dims 16 ks + 8 g .. +7 (k-step ks)
    e([I(f"s_add_u32 {T0}, {sr(S_KROW)}, {sr(S_K0)}")])              # first key row of the wave
    e(rows_bytes(T1, T2, T0))
    e(res64(S_RQ, "k", T1, T2, 32 * RB))
    e(res64(S_RO, "v", T1, T2, 32 * RB))
    e([I(f"v_and_b32 {vr(V_TMP)}, 31, {vr(V_LANE)}"),
       I(f"v_lshlrev_b32 {vr(V_TMP)}, 8, {vr(V_TMP)}"),                # c * 256
       I(f"v_lshrrev_b32 {vr(V_TMP + 1)}, 5, {vr(V_LANE)}"),
       I(f"v_lshl_add_u32 {vr(V_TMP)}, {vr(V_TMP + 1)}, 4, {vr(V_TMP)}")])   # + 16 g
    for ks in range(8):
        e(I(f"buffer_load_dwordx4 {vr(KF + 4 * ks, 4)}, {vr(V_TMP)}, {sr(S_RQ, 4)}, 0 offen "
            f"offset:{32 * ks}"))
    for ks in range(8):
        e(I(f"buffer_load_dwordx4 {vr(VF + 4 * ks, 4)}, {vr(V_TMP)}, {sr(S_RO, 4)}, 0 offen "
            f"offset:{32 * ks}"))
    # ---- per-lane LDS offsets
    # row reads (A of S/dP): row arow(c), chunk 4 m + 2 h + g  ->  RO[2 m + h]
    # transposing reads (B of dV/dK): rows tr + 4 h, chunk 4 m + tq, + 8 (lane & 1)
    C, G = V_TMP + 1, V_TMP + 2
    e([I(f"v_and_b32 {vr(C)}, 31, {vr(V_LANE)}"),
       I(f"v_lshrrev_b32 {vr(G)}, 5, {vr(V_LANE)}"),
       # arow(c) = (c & 0x13) | ((c & 4) << 1) | ((c & 8) >> 1)
       I(f"v_and_b32 {vr(V_TMP + 3)}, 0x13, {vr(C)}"),
       I(f"v_bfe_u32 {vr(V_TMP + 4)}, {vr(C)}, 2, 1"),
       I(f"v_lshl_or_b32 {vr(V_TMP + 3)}, {vr(V_TMP + 4)}, 3, {vr(V_TMP + 3)}"),
       I(f"v_bfe_u32 {vr(V_TMP + 4)}, {vr(C)}, 3, 1"),
       I(f"v_lshl_or_b32 {vr(V_TMP + 3)}, {vr(V_TMP + 4)}, 2, {vr(V_TMP + 3)}"),   # rr
       # swz key of rr: 4 (rr & 3) + ((rr >> 2) & 3)
       I(f"v_and_b32 {vr(V_TMP + 4)}, 3, {vr(V_TMP + 3)}"),
       I(f"v_bfe_u32 {vr(V_TMP + 5)}, {vr(V_TMP + 3)}, 2, 2"),
       I(f"v_lshl_or_b32 {vr(V_TMP + 4)}, {vr(V_TMP + 4)}, 2, {vr(V_TMP + 5)}"),
       I(f"v_lshlrev_b32 {vr(V_TMP + 3)}, 8, {vr(V_TMP + 3)}")])                   # rr * 256
    for m in range(4):
        for h in range(2):
            e([I(f"v_add_u32 {vr(V_TMP + 5)}, {4 * m + 2 * h}, {vr(G)}"),
               I(f"v_xor_b32 {vr(V_TMP + 5)}, {vr(V_TMP + 5)}, {vr(V_TMP + 4)}"),
               I(f"v_lshl_add_u32 {vr(RO + 2 * m + h)}, {vr(V_TMP + 5)}, 4, {vr(V_TMP + 3)}")])
    # tr = 8 g + ((lane & 15) >> 2), tq = 2 ((lane >> 4) & 1) + ((lane & 3) >> 1)
    e([I(f"v_bfe_u32 {vr(V_TMP + 3)}, {vr(V_LANE)}, 2, 2"),
       I(f"v_lshl_add_u32 {vr(V_TMP + 3)}, {vr(G)}, 3, {vr(V_TMP + 3)}"),          # tr
       I(f"v_bfe_u32 {vr(V_TMP + 4)}, {vr(V_LANE)}, 4, 1"),
       I(f"v_bfe_u32 {vr(V_TMP + 5)}, {vr(V_LANE)}, 1, 1"),
       I(f"v_lshl_or_b32 {vr(V_TMP + 4)}, {vr(V_TMP + 4)}, 1, {vr(V_TMP + 5)}"),   # tq
       I(f"v_and_b32 {vr(V_TMP + 5)}, 1, {vr(V_LANE)}"),
       I(f"v_lshlrev_b32 {vr(V_TMP + 5)}, 3, {vr(V_TMP + 5)}")])                   # 8 (lane & 1)
    for h in range(2):
        R, K = V_TMP + 6, V_TMP + 7
        e([I(f"v_add_u32 {vr(R)}, {4 * h}, {vr(V_TMP + 3)}"),
           I(f"v_and_b32 {vr(K)}, 3, {vr(R)}"),
           I(f"v_bfe_u32 {vr(C)}, {vr(R)}, 2, 2"),
           I(f"v_lshl_or_b32 {vr(K)}, {vr(K)}, 2, {vr(C)}"),                        # swz key
           I(f"v_lshlrev_b32 {vr(R)}, 8, {vr(R)}"),
           I(f"v_add_u32 {vr(R)}, {vr(R)}, {vr(V_TMP + 5)}")])
        for m in range(4):
            e([I(f"v_add_u32 {vr(C)}, {4 * m}, {vr(V_TMP + 4)}"),
               I(f"v_xor_b32 {vr(C)}, {vr(C)}, {vr(K)}"),
               I(f"v_lshl_add_u32 {vr(TO + 2 * m + h)}, {vr(C)}, 4, {vr(R)}")])
    # bias reads: rows 8 g (+ 16) of a sub-block: 32 g bytes; dS store: 16 lane
    e([I(f"v_lshrrev_b32 {vr(G)}, 5, {vr(V_LANE)}"),
       I(f"v_lshlrev_b32 {vr(V_LDB)}, 5, {vr(G)}"),
       I(f"v_add_u32 {vr(V_LDB)}, {T_LD}, {vr(V_LDB)}"),
       I(f"v_lshlrev_b32 {vr(V_DSOFF)}, 4, {vr(V_LANE)}")])
    # transfers: instruction i of wave w covers rows 32 w + 4 i + (lane >> 4) (LDS KiB 8 w + i);
    # slot lane & 15 holds logical chunk (lane & 15) ^ swz(4 (i & 3) + (lane >> 4)), i.e.
    # (lane & 15) ^ (4 (lane >> 4) + (i & 3)). The instruction offset 1024 (i & 3) moves the LDS
    # and the global address alike, M0 + 4 KiB and soffset 4096 cover i >= 4, so the lane
    # offset of instructions k and k + 4 is (32 w + (lane >> 4)) * 256 + 16 chunk.
    e([I(f"v_lshrrev_b32 {vr(V_TMP + 3)}, 4, {vr(V_LANE)}"),                      # lane >> 4
       I(f"s_lshl_b32 {T0}, {sr(S_WAVE)}, 5"),
       I(f"v_add_u32 {vr(V_TMP + 4)}, {T0}, {vr(V_TMP + 3)}"),
       I(f"v_lshlrev_b32 {vr(V_TMP + 4)}, 8, {vr(V_TMP + 4)}"),                    # row bytes
       I(f"v_lshlrev_b32 {vr(V_TMP + 5)}, 2, {vr(V_TMP + 3)}"),
       I(f"v_and_b32 {vr(V_TMP + 6)}, 15, {vr(V_LANE)}")])
    for k in range(4):
        e([I(f"v_add_u32 {vr(V_TMP + 7)}, {k}, {vr(V_TMP + 5)}"),
           I(f"v_xor_b32 {vr(V_TMP + 7)}, {vr(V_TMP + 7)}, {vr(V_TMP + 6)}"),        # chunk
           I(f"v_lshl_add_u32 {vr(xoff(k))}, {vr(V_TMP + 7)}, 4, {vr(V_TMP + 4)}")])
    # bias transfer (wave 0): lanes 0..31 -LSE rows 4 l .. (16 bytes each), lanes 32..63 the
    # -delta rows, rows * 4 bytes further on
    e([I(f"v_and_b32 {vr(V_TMP + 3)}, 31, {vr(V_LANE)}"),
       I(f"v_lshlrev_b32 {vr(V_LDOFF)}, 4, {vr(V_TMP + 3)}"),
       I(f"v_cmp_le_u32 vcc, 32, {vr(V_LANE)}", reads=[f"v{V_LANE}"], writes=["vcc"]),
       I(f"s_lshl_b32 {T0}, {arg('rows')}, 2"),
       I(f"v_mov_b32 {vr(V_TMP + 4)}, {T0}"),
       I(f"v_cndmask_b32 {vr(V_TMP + 4)}, 0, {vr(V_TMP + 4)}, vcc",
         reads=[f"v{V_TMP + 4}", "vcc"], writes=[f"v{V_TMP + 4}"]),
       I(f"v_add_u32 {vr(V_LDOFF)}, {vr(V_LDOFF)}, {vr(V_TMP + 4)}")])
    # ---- dK = dV = 0 (eight MFMAs of zero operands)
    e([I(f"v_mov_b32 {vr(V_TMP + i)}, 0") for i in range(4)])
    for blk in range(8):
        e(I(f"{MF()} {ar(16 * blk, 16)}, {vr(V_TMP, 4)}, {vr(V_TMP, 4)}, 0"))
    # ---- tile 0 into stage 0
    # tile order: query tiles outer, the group's heads inner; the first half of the key blocks
    # sweeps the queries downwards from the last tile, the second half upwards from its
    # diagonal. Under a causal mask the heavy first half runs first, one workgroup per CU, and a
    # second-half workgroup starts on the CU whose first-half workgroup ended, so at any time
    # the running workgroups of one (batch, kv head) read the same query tile (a shared L2).
    e([I(f"s_mov_b32 {sr(S_J)}, 0"), I(f"s_mov_b32 {sr(S_HH)}, 0"),
       I(f"s_lshl_b32 {T0}, {sr(S_KB)}, 8"),
       I(f"s_sub_u32 {T1}, {arg('seq')}, 128"),
       I(f"s_mov_b32 {sr(S_DQ)}, 128"),
       I(f"s_cmp_lt_u32 {T0}, {arg('seq')}"),
       I(f"s_cselect_b32 {sr(S_QT)}, {T1}, {sr(S_QSTART)}"),
       I(f"s_cselect_b32 {sr(S_DQ)}, -128, {sr(S_DQ)}"),
       I(f"s_mov_b32 {sr(S_STAGE)}, 0"), I(f"s_mov_b32 {sr(S_CUR)}, 0"),
       I(f"s_mov_b32 {sr(S_CURL)}, 0")])
    # resource bytes of the transfers: a whole tile of Q / dO; the bias resource starts at the
    # tile's first row of the -LSE array and reaches the -delta rows, rows * 4 bytes on
    e([I(f"s_mov_b32 {sr(S_NRQ)}, {128 * RB}"),
       I(f"s_lshl_b32 {sr(S_NRL)}, {arg('rows')}, 2"),
       I(f"s_add_u32 {sr(S_NRL)}, {sr(S_NRL)}, 512")])
    e(transfer_setup(sr(S_HH), sr(S_QT), 0, sr(S_NRQ), sr(S_NRL)))
    for grp in transfer_items():
        e(grp)
    e([I("s_waitcnt vmcnt(0)"), I("s_barrier")])


def transfer_setup(hh_sgpr, qt_sgpr, stage, nrec_q, nrec_l) -> list:
    """Resources and LDS destinations of the transfers of tile (hh, qt) into LDS stage `stage`
    (an SGPR or a constant); nrec_q / nrec_l: resource bytes (SGPRs; 0 for a tile past the
    last, whose transfers then read nothing and write zeros to the free stage)."""
    T0, T1, T2, T3 = (sr(S_T0), sr(S_T1), sr(S_T2), sr(S_T3))
    out = [I(f"s_mul_i32 {T0}, {hh_sgpr}, {arg('seq')}"),
           I(f"s_add_u32 {T0}, {T0}, {sr(S_QH0)}"),
           I(f"s_add_u32 {T0}, {T0}, {qt_sgpr}")]                      # first row of the tile
    out += rows_bytes(T1, T2, T0)
    out += res64(S_RQ, "q", T1, T2, nrec_q)
    out += res64(S_RO, "dout", T1, T2, nrec_q)
    out += [I(f"s_lshl_b32 {T1}, {T0}, 2"),
            I(f"s_add_u32 {sr(S_RL)}, {arg('ld')}, {T1}"),
            I(f"s_addc_u32 {sr(S_RL + 1)}, {arg('ld', True)}, 0"),
            I(f"s_and_b32 {sr(S_RL + 1)}, {sr(S_RL + 1)}, 0xffff"),
            I(f"s_mov_b32 {sr(S_RL + 3)}, 0x20000"),
            I(f"s_lshl_b32 {sr(S_XB)}, {sr(S_WAVE)}, 13"),
            I(f"s_add_u32 {sr(S_XB)}, {sr(S_XB)}, {stage}"),
            I(f"s_mov_b32 {sr(S_XSOFF)}, 0x1000"),
            I(f"s_add_u32 {sr(S_XBL)}, {stage}, {T_LD}"),
            # the biases: one instruction of wave 0; the other waves read no bytes
            I(f"s_mov_b32 {T0}, {DUMMY}"),
            I(f"s_cmp_eq_u32 {sr(S_WAVE)}, 0"),
            I(f"s_cselect_b32 {sr(S_XBL)}, {sr(S_XBL)}, {T0}"),
            I(f"s_cselect_b32 {sr(S_RL + 2)}, {nrec_l}, 0")]
    return out


def transfer_items() -> list:
    """The transfer instructions after transfer_setup, in groups that can be spread over a
    tile's MFMAs: 8 Q and 8 dO instructions per wave (4 rows each: rows 32 w + 4 i + lane / 16,
    the same per-lane offsets for both; one M0 per four instructions), then the biases."""
    out = []
    for rs, region in ((S_RQ, 0), (S_RO, T_DO)):
        for i in range(8):
            grp = []
            if i % 4 == 0:
                grp.append(I(f"s_add_u32 m0, {sr(S_XB)}, {region + 4096 * (i // 4)}",
                             writes=["m0"], reads=[f"s{S_XB}"]))
            soff = "0" if i < 4 else sr(S_XSOFF)
            grp.append(I(f"buffer_load_dwordx4 {vr(xoff(i % 4))}, {sr(rs, 4)}, {soff} offen "
                         f"offset:{1024 * (i % 4)} lds"))
            out.append(grp)
    out.append([I(f"s_mov_b32 m0, {sr(S_XBL)}", writes=["m0"], reads=[f"s{S_XBL}"]),
                I(f"buffer_load_dwordx4 {vr(V_LDOFF)}, {sr(S_RL, 4)}, 0 offen lds")])
    return out


# --------------------------------------------------------------------------- the tile loop
def tile_setup() -> list:
    """Per tile: first active sub-block s0 (the wave's diagonal on the first tile of a head
    under a causal mask), the read offsets moved to this tile's stage and s0, the dS store
    resource of this tile. SCC on exit: the tile holds the causal diagonal."""
    T0, T1, T2, T3 = (sr(S_T0), sr(S_T1), sr(S_T2), sr(S_T3))
    out = [# diag = causal && qt == qstart; s0 = diag ? wave : 0
           I(f"s_cmp_eq_u32 {sr(S_QT)}, {sr(S_QSTART)}"),
           I(f"s_cselect_b32 {sr(S_S0)}, {sr(S_WAVE)}, 0"),
           I(f"s_cmp_eq_u32 {arg('causal')}, 0"),
           I(f"s_cselect_b32 {sr(S_S0)}, 0, {sr(S_S0)}"),
           # read offsets: stage + s0 * SUB
           I(f"s_mul_i32 {T0}, {sr(S_S0)}, {SUB}"),
           I(f"s_add_u32 {T0}, {T0}, {sr(S_STAGE)}"),
           I(f"s_sub_u32 {T1}, {T0}, {sr(S_CUR)}"),
           I(f"s_mov_b32 {sr(S_CUR)}, {T0}")]
    out += [I(f"v_add_u32 {vr(RO + i)}, {T1}, {vr(RO + i)}") for i in range(8)]
    out += [I(f"v_add_u32 {vr(TO + i)}, {T1}, {vr(TO + i)}") for i in range(8)]
    out += [I(f"s_lshl_b32 {T0}, {sr(S_S0)}, 7"),
            I(f"s_add_u32 {T0}, {T0}, {sr(S_STAGE)}"),
            I(f"s_sub_u32 {T1}, {T0}, {sr(S_CURL)}"),
            I(f"s_mov_b32 {sr(S_CURL)}, {T0}"),
            I(f"v_add_u32 {vr(V_LDB)}, {T1}, {vr(V_LDB)}")]
    # dS group of (head, qt / 128, k0 / 32): ((b Hq + kvh G + hh) gph + base(t) + k0 / 32) * 8 KiB
    # with base(t) = causal ? 2 t (t + 1) : t nb; + s0 * 2 KiB
    out += [I(f"s_mul_i32 {T0}, {sr(S_B)}, {arg('q_heads')}"),
            I(f"s_mul_i32 {T1}, {sr(S_KVH)}, {arg('group')}"),
            I(f"s_add_u32 {T0}, {T0}, {T1}"),
            I(f"s_add_u32 {T0}, {T0}, {sr(S_HH)}"),
            I(f"s_mul_i32 {T0}, {T0}, {arg('ds_gph')}"),
            I(f"s_lshr_b32 {T1}, {sr(S_QT)}, 7"),                          # t
            I(f"s_add_u32 {T2}, {T1}, 1"),
            I(f"s_mul_i32 {T2}, {T2}, {T1}"),
            I(f"s_lshl_b32 {T2}, {T2}, 1"),                                # 2 t (t + 1)
            I(f"s_mul_i32 {T1}, {T1}, {arg('ds_nb')}"),                    # t nb
            I(f"s_cmp_eq_u32 {arg('causal')}, 0"),
            I(f"s_cselect_b32 {T2}, {T1}, {T2}"),
            I(f"s_add_u32 {T0}, {T0}, {T2}"),
            I(f"s_lshr_b32 {T1}, {sr(S_K0)}, 5"),
            I(f"s_add_u32 {T0}, {T0}, {T1}"),
            I(f"s_lshl_b32 {T0}, {T0}, 13"),
            I(f"s_lshl_b32 {T1}, {sr(S_S0)}, 11"),
            I(f"s_add_u32 {T0}, {T0}, {T1}"),                              # byte offset
            I(f"s_add_u32 {sr(S_RD)}, {arg('ds')}, {T0}"),
            I(f"s_addc_u32 {sr(S_RD + 1)}, {arg('ds', True)}, 0"),
            I(f"s_and_b32 {sr(S_RD + 1)}, {sr(S_RD + 1)}, 0xffff"),
            I(f"s_sub_u32 {sr(S_RD + 2)}, {arg('ds_bytes')}, {T0}"),
            I(f"s_mov_b32 {sr(S_RD + 3)}, 0x20000"),
            # SCC = diagonal tile (s0 came from the wave index on a causal first tile)
            I(f"s_cmp_eq_u32 {sr(S_QT)}, {sr(S_QSTART)}"),
            I(f"s_cselect_b32 {T0}, 1, 0"),
            I(f"s_cmp_eq_u32 {arg('causal')}, 0"),
            I(f"s_cselect_b32 {T0}, 0, {T0}"),
            I(f"s_cmp_eq_u32 {T0}, 1")]
    return out


# --------------------------------------------------------------------------- one tile
ISSUE_COST = {"trans": 2}


def diag_masks(t):
    """Lanes whose key c exceeds the query kidx(g, t) of register t on the diagonal block."""
    def m(k):
        return (0xFFFFFFFF << (k + 1)) & 0xFFFFFFFF if k + 1 < 32 else 0
    return m(kidx(0, t)), m(kidx(1, t))


def softmax(i: int, masked: bool) -> list:
    """P = exp2(c2 S'), dS = P dP' of local sub-block i (accumulators of parity i & 1), packed
    into PF / DF (register 4 s + j holds rows 8 s + 2 j, + 1 of the lane's key)."""
    S, D = SACC[i & 1], DACC[i & 1]
    out = []
    c2 = arg("c2")
    for t in range(0, 16, 2):
        out += [I(f"v_mul_f32 {vr(S + t)}, {c2}, {vr(S + t)}"),
                I(f"v_mul_f32 {vr(S + t + 1)}, {c2}, {vr(S + t + 1)}"),
                I(f"v_exp_f32 {vr(S + t)}, {vr(S + t)}"),
                I(f"v_exp_f32 {vr(S + t + 1)}, {vr(S + t + 1)}")]
        if masked:
            for tt in (t, t + 1):
                lo, hi = diag_masks(tt)
                out += [I(f"s_mov_b32 {sr(S_MASK)}, 0x{lo:x}"),
                        I(f"s_mov_b32 {sr(S_MASK + 1)}, 0x{hi:x}"),
                        I(f"v_cndmask_b32_e64 {vr(S + tt)}, {vr(S + tt)}, 0, {sr(S_MASK, 2)}",
                          reads=[f"v{S + tt}", f"s{S_MASK}", f"s{S_MASK + 1}"],
                          writes=[f"v{S + tt}"])]
        out += [I(f"v_mul_f32 {vr(D + t)}, {vr(S + t)}, {vr(D + t)}"),
                I(f"v_mul_f32 {vr(D + t + 1)}, {vr(S + t + 1)}, {vr(D + t + 1)}")]
        reg = 4 * (t >> 3) + ((t & 7) >> 1)
        out += [I(f"{CVT()} {vr(PF + reg)}, {vr(S + t)}, {vr(S + t + 1)}"),
                I(f"{CVT()} {vr(DF + reg)}, {vr(D + t)}, {vr(D + t + 1)}")]
    return out


def ds_store(i: int) -> list:
    """dS of local sub-block i into its 2 KiB block of the tile's dS group (non-temporal)."""
    return [I(f"s_mov_b32 {sr(S_SOFF)}, {2048 * i}"),
            I(f"buffer_store_dwordx4 {vr(DF, 4)}, {vr(V_DSOFF)}, {sr(S_RD, 4)}, {sr(S_SOFF)} "
              f"offen nt"),
            I(f"buffer_store_dwordx4 {vr(DF + 4, 4)}, {vr(V_DSOFF)}, {sr(S_RD, 4)}, {sr(S_SOFF)} "
              f"offen offset:1024 nt")]


def body(gen: Gen, n: int, diag: bool, xfer: list):
    """The n active sub-blocks of a tile (the first on the causal diagonal when diag): MFMA
    sequence chain(0), [chain(1), dvdk(0)], ..., [dvdk(n-1)]; chain(i) = S'/dP' of sub-block i,
    dvdk(i) = its dV/dK products; softmax(i) spread over chain(i+1)."""
    e = gen.emit
    ml = []   # (kind, i, k)
    ml += [("c", 0, k) for k in range(16)]
    ranges = {}
    for i in range(n):
        start = len(ml)
        if i + 1 < n:
            ml += [("c", i + 1, k) for k in range(16)]
        ranges[i] = (start, len(ml))          # where softmax(i) is spread (may be empty)
        ml += [("d", i, k) for k in range(16)]
    # bias loads of sub-block i: before chain(i); for i >= 1 after MFMA 6 of chain(i - 1)
    bias_ids = {}

    def bias_loads(i):
        ids = []
        base = i * 128
        for which, reg, off in (("l", LB, 0), ("d", DB, 512)):
            for hlf in range(2):
                for q in range(2):
                    ids.append(gen.ds_issue(
                        f"ds_read_b128 {vr(reg + 8 * hlf + 4 * q, 4)}, {vr(V_LDB)} "
                        f"offset:{base + off + 64 * hlf + 16 * q}"))
        bias_ids[i] = ids
    chain_pos = {}
    for idx, (kind, i, k) in enumerate(ml):
        if kind == "c":
            chain_pos.setdefault(i, idx)
    # operand rings
    reads_a = [idx for idx, x in enumerate(ml) if x[0] == "c"]
    reads_b = [idx for idx, x in enumerate(ml) if x[0] == "d"]
    issued = {}
    na = nb = 0
    emitted = -1

    def issue(budget):
        nonlocal na, nb
        cnt = 0
        while cnt < budget:
            progressed = False
            if na < len(reads_a):
                j = na
                if j < RA or reads_a[j - RA] <= emitted:
                    idx = reads_a[j]
                    _, i, k = ml[idx]
                    ks = k >> 1
                    off = i * SUB + (T_DO if k & 1 else 0)
                    slot = a_slot(j)
                    issued[idx] = [gen.ds_issue(f"ds_read_b128 {vr(slot, 4)}, {vr(RO + ks)} "
                                                f"offset:{off}")]
                    na += 1
                    cnt += 1
                    progressed = True
            if cnt < budget and nb < len(reads_b):
                j = nb
                if j < RBN or reads_b[j - RBN] <= emitted:
                    idx = reads_b[j]
                    _, i, k = ml[idx]
                    mb, s_, is_dk = k >> 2, (k >> 1) & 1, k & 1
                    off = i * SUB + 16 * s_ * RB + (0 if is_dk else T_DO)
                    slot = BRING + 4 * (j % RBN)
                    issued[idx] = [
                        gen.ds_issue(f"ds_read_b64_tr_b16 {vr(slot, 2)}, {vr(TO + 2 * mb)} "
                                     f"offset:{off}"),
                        gen.ds_issue(f"ds_read_b64_tr_b16 {vr(slot + 2, 2)}, "
                                     f"{vr(TO + 2 * mb + 1)} offset:{off}")]
                    nb += 1
                    cnt += 1
                    progressed = True
            if not progressed:
                break

    # the first sub-block's biases, then fill the rings
    bias_loads(0)
    issue(RA + RBN)
    streams = {}
    stores = {}
    for i in range(n):
        streams[i] = softmax(i, diag and i == 0)
        st = ds_store(i)
        stores[i] = [st[:2], st[2:]]
    # the next tile's transfers: one group every `stride` MFMAs from the second on, over the
    # first half of the tile (a burst of them stalls the issue behind the memory pipeline)
    xfer = list(xfer)
    stride = max(1, min(4, (len(ml) // 2) // max(1, len(xfer))))
    xfer_at = {1 + stride * k: grp for k, grp in enumerate(xfer)}
    vm_order = []     # "x" (transfer) / "s" (dS store), in issue order
    pending_stream = []     # (remaining items, cost, first idx allowed)
    for idx, (kind, i, k) in enumerate(ml):
        # softmax(i) must be out before dvdk(i) starts
        if kind == "d" and k == 0 and streams.get(i):
            for x in streams.pop(i):
                e(x)
        if kind == "c" and k == 0:
            gen.ds_wait_for(bias_ids[i])
        gen.ds_wait_for(issued[idx])
        if kind == "c":
            ks = k >> 1
            acc = (DACC if k & 1 else SACC)[i & 1]
            frag = (VF if k & 1 else KF) + 4 * ks
            src = vr((DB if k & 1 else LB), 16) if ks == 0 else vr(acc, 16)
            slot = a_slot(reads_a.index(idx))
            ins = I(f"{MF()} {vr(acc, 16)}, {vr(slot, 4)}, {vr(frag, 4)}, "
                    f"{src}")
            ins.srcc_chain = ks != 0
        else:
            mb, s_, is_dk = k >> 2, (k >> 1) & 1, k & 1
            acc = (A_DK if is_dk else A_DV) + 16 * mb
            a_op = (DF if is_dk else PF) + 4 * s_
            slot = BRING + 4 * (reads_b.index(idx) % RBN)
            ins = I(f"{MF()} {ar(acc, 16)}, {vr(a_op, 4)}, {vr(slot, 4)}, "
                    f"{ar(acc, 16)}")
            ins.srcc_chain = True
        e(ins)
        emitted = idx
        if idx in xfer_at:
            e(xfer_at.pop(idx))
            vm_order.append("x")
        # the dS stores of sub-block i after its third and ninth dV/dK MFMAs
        if kind == "d" and k in (2, 8):
            e(stores[i].pop(0))
            vm_order.append("s")
        issue(2)
        # next sub-block's biases once this chain's first MFMAs have read the bias registers
        if kind == "c" and k == 6 and i + 1 < n:
            bias_loads(i + 1)
        # spread softmax(i) over the MFMAs of chain(i + 1)
        for si, (a0, a1) in ranges.items():
            if a0 <= idx < a1 and streams.get(si):
                items = streams[si]
                left = sum(ISSUE_COST.get(x.kind, 1) for x in items)
                slots = a1 - idx
                budget = (left + slots - 1) // slots
                spent = 0
                while items and spent < budget:
                    x = items.pop(0)
                    spent += ISSUE_COST.get(x.kind, 1)
                    e(x)
    for i in sorted(streams):
        for x in streams[i]:
            e(x)
    for k in sorted(xfer_at):
        e(xfer_at[k])
        vm_order.append("x")
    assert not any(stores.values())
    gen.ds_wait_all()
    # the dS stores issued after the last transfer may stay in flight; the transfers must land
    last_x = max(i for i, v in enumerate(vm_order) if v == "x") if "x" in vm_order else -1
    e(I(f"s_waitcnt vmcnt({len(vm_order) - 1 - last_x})"))


# --------------------------------------------------------------------------- epilogue
EP_ROWB = 272                  # staging row of 128 bf16, padded
EP_TENSOR = 32 * EP_ROWB       # one tensor of the wave (32 keys)
EP_WAVE = 2 * EP_TENSOR


def epilogue(gen: Gen):
    """dV and dK * scale as bf16 rows: register r of lane (g, c) holds key 8 (r / 4) + 4 g + r % 4
    of the wave, dim 32 mb + c; written to LDS one element at a time, read back as 16-byte
    row pieces (16 lanes per 256-byte row) and stored with whole-row coalesced stores."""
    e = gen.emit
    T0, T1, T2 = sr(S_T0), sr(S_T1), sr(S_T2)
    C, G = V_TMP, V_TMP + 1
    # write base: wave region + 4 g rows + 2 c; read base: (lane >> 4) rows + 16 (lane & 15)
    e([I(f"s_mul_i32 {T0}, {sr(S_WAVE)}, {EP_WAVE}"),
       I(f"v_and_b32 {vr(C)}, 31, {vr(V_LANE)}"),
       I(f"v_lshrrev_b32 {vr(G)}, 5, {vr(V_LANE)}"),
       I(f"v_mul_u32_u24 {vr(V_EPW)}, {4 * EP_ROWB}, {vr(G)}"),
       I(f"v_lshl_add_u32 {vr(V_EPW)}, {vr(C)}, 1, {vr(V_EPW)}"),
       I(f"v_add_u32 {vr(V_EPW)}, {T0}, {vr(V_EPW)}"),
       I(f"v_lshrrev_b32 {vr(G)}, 4, {vr(V_LANE)}"),
       I(f"v_and_b32 {vr(C)}, 15, {vr(V_LANE)}"),
       I(f"v_mul_u32_u24 {vr(V_EPR)}, {EP_ROWB}, {vr(G)}"),
       I(f"v_lshl_add_u32 {vr(V_EPR)}, {vr(C)}, 4, {vr(V_EPR)}"),
       I(f"v_add_u32 {vr(V_EPR)}, {T0}, {vr(V_EPR)}"),
       I(f"v_lshlrev_b32 {vr(V_EPG)}, 8, {vr(G)}"),
       I(f"v_lshl_add_u32 {vr(V_EPG)}, {vr(C)}, 4, {vr(V_EPG)}")])
    X = SACC[0]           # 16 converted values
    for tensor, abase, scaled in ((0, A_DV, False), (1, A_DK, True)):
        for mb in range(4):
            e([I(f"v_accvgpr_read_b32 {vr(X + r)}, {ar(abase + 16 * mb + r)}") for r in range(16)])
            if scaled:
                e([I(f"v_mul_f32 {vr(X + r)}, {arg('scale')}, {vr(X + r)}") for r in range(16)])
            e([I(f"{CVT()} {vr(X + r)}, {vr(X + r)}, 0") for r in range(16)])
            for r in range(16):
                off = tensor * EP_TENSOR + (8 * (r >> 2) + (r & 3)) * EP_ROWB + 64 * mb
                e(I(f"ds_write_b16 {vr(V_EPW)}, {vr(X + r)} offset:{off}"))
    e(I("s_waitcnt lgkmcnt(0)"))
    # rows 4 i + (lane >> 4) of the wave's 32 keys; 8 reads per tensor
    D0 = SACC[0]          # 64 registers: SACC, DACC
    for tensor, name in ((0, "dv"), (1, "dk")):
        for i in range(8):
            e(I(f"ds_read_b128 {vr(D0 + 4 * i, 4)}, {vr(V_EPR)} "
                f"offset:{tensor * EP_TENSOR + 4 * i * EP_ROWB}"))
        e([I(f"s_add_u32 {T0}, {sr(S_KROW)}, {sr(S_K0)}")])
        e(rows_bytes(T1, T2, T0))
        e(res64(S_RQ, name, T1, T2, 32 * RB))
        e(I("s_waitcnt lgkmcnt(0)"))
        for i in range(8):
            e([I(f"s_mov_b32 {sr(S_SOFF)}, {4 * i * RB}"),
               I(f"buffer_store_dwordx4 {vr(D0 + 4 * i, 4)}, {vr(V_EPG)}, {sr(S_RQ, 4)}, "
                 f"{sr(S_SOFF)} offen")])
        # the next tensor's reads overwrite these registers: wait for the stores to take them
        e(I("s_waitcnt vmcnt(0)"))
    e(I("s_endpgm"))


# --------------------------------------------------------------------------- the program
def build() -> Gen:
    gen = Gen()
    b_setup = gen.new_block("setup")
    setup(gen)
    b_tile = gen.new_block("tile", [b_setup])
    e = gen.emit
    T0 = sr(S_T0)
    e([I(".Ltile:"),
       # next tile: the next head of the group, wrapping to the next query tile
       I(f"s_add_u32 {sr(S_NHH)}, {sr(S_HH)}, 1"),
       I(f"s_mov_b32 {sr(S_NQ)}, {sr(S_QT)}"),
       I(f"s_cmp_ge_u32 {sr(S_NHH)}, {arg('group')}"),
       I(f"s_cselect_b32 {sr(S_NHH)}, 0, {sr(S_NHH)}"),
       I(f"s_cselect_b32 {T0}, {sr(S_DQ)}, 0"),
       I(f"s_add_u32 {sr(S_NQ)}, {sr(S_NQ)}, {T0}"),
       I(f"s_sub_u32 {sr(S_XST)}, {STAGE}, {sr(S_STAGE)}"),
       # past the last tile the transfers read nothing
       I(f"s_add_u32 {T0}, {sr(S_J)}, 1"),
       I(f"s_cmp_lt_u32 {T0}, {sr(S_NT)}"),
       I(f"s_cselect_b32 {sr(S_XNQ)}, {sr(S_NRQ)}, 0"),
       I(f"s_cselect_b32 {sr(S_XNL)}, {sr(S_NRL)}, 0")])
    e(transfer_setup(sr(S_NHH), sr(S_NQ), sr(S_XST), sr(S_XNQ), sr(S_XNL)))
    b_nox = b_tile
    e(tile_setup())
    e(I("s_cbranch_scc1 .Ldiag"))
    ends = []
    gen.new_block("full", [b_nox])
    body(gen, 4, False, transfer_items())
    e(I("s_branch .Ltend"))
    ends.append(gen.cur)
    b_disp = gen.new_block("diag", [b_nox])
    e([I(".Ldiag:"),
       I(f"s_cmp_eq_u32 {sr(S_WAVE)}, 0"), I("s_cbranch_scc1 .Ld4"),
       I(f"s_cmp_eq_u32 {sr(S_WAVE)}, 1"), I("s_cbranch_scc1 .Ld3"),
       I(f"s_cmp_eq_u32 {sr(S_WAVE)}, 2"), I("s_cbranch_scc1 .Ld2")])
    for n in (1, 4, 3, 2):
        gen.new_block(f"d{n}", [b_disp])
        if n != 1:
            e(I(f".Ld{n}:"))
        body(gen, n, True, transfer_items())
        e(I("s_branch .Ltend"))
        ends.append(gen.cur)
    b_end = gen.new_block("tend", ends)
    e([I(".Ltend:"),
       I("s_barrier"),
       I(f"s_mov_b32 {sr(S_HH)}, {sr(S_NHH)}"),
       I(f"s_mov_b32 {sr(S_QT)}, {sr(S_NQ)}"),
       I(f"s_mov_b32 {sr(S_STAGE)}, {sr(S_XST)}"),
       I(f"s_add_u32 {sr(S_J)}, {sr(S_J)}, 1"),
       I(f"s_cmp_lt_u32 {sr(S_J)}, {sr(S_NT)}"),
       I("s_cbranch_scc1 .Ltile")])
    b_tile.preds.append(b_end)
    gen.new_block("epilogue", [b_end])
    epilogue(gen)
    return gen


# --------------------------------------------------------------------------- hazards
_base_required = P.required


def required(prev, cur) -> int:
    """The prefill generator's rules plus two this kernel's schedule meets: a VALU or memory
    write of a register an MFMA read as its accumulator input (write-after-read; 11 wait states
    covers the 8-pass 32x32x16 MFMA), and a VALU write of the data registers of a store wider
    than 64 bits (2)."""
    need = _base_required(prev, cur)
    if cur.kind in ("label", "nop"):
        return need
    if prev.kind == "mfma" and cur.kind in ("valu", "trans", "permlane", "ds", "vmem"):
        parts = [x.strip() for x in prev.text.split(None, 1)[1].split(",")]
        srcc = set(P.regs_in(parts[3])) if len(parts) > 3 else set()
        if srcc & cur.writes:
            need = max(need, 11)
    if (prev.kind == "vmem" and prev.text.startswith(("buffer_store_dwordx3",
                                                      "buffer_store_dwordx4"))
            and cur.kind in ("valu", "trans", "permlane")):
        data = set(P.regs_in(prev.text.split(None, 1)[1].split(",")[0]))
        if data & cur.writes:
            need = max(need, 2)
    return need


def render() -> str:
    P.required = required
    try:
        global F16, KERNEL
        out = []
        for f16, name, prefix in ((False, KERNEL_BF16, ""), (True, KERNEL_F16, "H")):
            F16, KERNEL = f16, name
            out.append((build(), name, prefix, {"num_vgpr": NUM_VGPR, "num_agpr": NUM_AGPR,
                                                "num_sgpr": NUM_SGPR, "lds_bytes": LDS_BYTES,
                                                "arg_bytes": ARG_BYTES}))
        return P.render(out)
    finally:
        F16, KERNEL = False, KERNEL_BF16
        P.required = _base_required


def header(path: str):
    lines = ["// Generated by gen_bwd_a64.py: kernel-argument layout of fa_bwd_dkdv_a64_bf16.",
             "#pragma once", f"#define FA_BWD_A64_ARG_BYTES {ARG_BYTES}",
             f"#define FA_BWD_A64_LDS_BYTES {LDS_BYTES}",
             f'#define FA_BWD_A64_KERNEL "{KERNEL_BF16}"',
             f'#define FA_BWD_A64_KERNEL_F16 "{KERNEL_F16}"']
    for n, off, sz in ARGS:
        lines.append(f"#define FA_BWD_A64_OFF_{n.upper()} {off}")
    open(path, "w").write("\n".join(lines) + "\n")


def blob(co_path: str, out_cpp: str):
    data = open(co_path, "rb").read()
    rows = [", ".join(f"0x{b:02x}" for b in data[i:i + 16]) for i in range(0, len(data), 16)]
    text = ("// Generated by gen_bwd_a64.py --blob: the assembled gfx950 code object of "
            "fa_bwd_dkdv_a64_bf16 and fa_bwd_dkdv_a64_f16.\n#include <stddef.h>\nnamespace fa {\n"
            "extern const unsigned char kBwdA64Co[] = {\n" + ",\n".join(rows) +
            f"\n}};\nextern const size_t kBwdA64CoSize = {len(data)};\n}}  // namespace fa\n")
    open(out_cpp, "w").write(text)


def main():
    if sys.argv[1] == "--blob":
        blob(sys.argv[2], sys.argv[3])
        return
    open(sys.argv[1], "w").write(render())
    header(sys.argv[2])


if __name__ == "__main__":
    main()
