#!/usr/bin/env python3
"""Generates the gfx950 assembly of the 16-bit prefill kernel `fa_prefill_a64` (64 query rows per
wave, one wave per SIMD) and the header that fixes its kernel-argument layout.

Usage: gen_prefill_a64.py OUT.s OUT_ARGS.h

Why assembly: a wave that holds 64 query rows keeps O^T (128 accumulators) and the rotated Q^T
operands (64 registers) resident in AGPRs, the scores of two 32-key half-tiles in VGPRs, and reads
every K and V^T operand once for two MFMAs (half the LDS bytes per MFMA of a 32-row wave). The
compiler cannot hold that register layout (it moves accumulators through VGPRs), so the kernel is
written here, with every register fixed and the instruction order chosen by the schedule below.

Math (forward_reference, src/lib.rs:454-520; RoPE rotated_pair, src/rotary_grouped.rs:37-50):
online softmax with running max m, running sum l, O accumulated with rescale alpha =
exp2((m_old - m_new) * scale * log2 e), LSE = m * scale + ln l. The running max only moves when a
half-tile's max exceeds it by more than 2^8 (in exp2 units): probabilities stay <= 2^8 and O, l
stay consistent, so the final O / l and LSE are exact either way.

Layout of the work (per workgroup of 4 waves = 256 query rows of one (batch, kv head)):
  row = t * group + head   (every query head of a GQA group shares each K/V tile)
  wave w holds rows r0 + 64 w .. +63 as two 32-row blocks rb = 0, 1; lane l holds row l % 32
  of each block; g = l / 32 selects which 8 of every 16 keys (dims) the lane supplies.
Per 32-key half-tile h (the pipeline unit):
  S^T[32 keys x 32 rows] (rb) = K_perm . Q^T(rb)   v_mfma_f32_32x32x16_bf16, A = K from LDS,
                                                   B = Q^T from AGPRs, 8 k-steps of 16 dims
  P^T = exp2(S * c2 - m * c2) packed to bf16        (every value a lane holds is its own row;
                                                   the f16 kernels: f16 MFMAs and packing)
  O^T[128 dims x 32 rows] (rb) += V^T . P^T         A = V^T from LDS (ds_read_b64_tr_b16),
                                                   B = P^T from VGPRs, O in AGPRs
K rows are fed in a permuted order (bits 2 and 3 of the row swapped) so that accumulator i of a
lane holds key 16 (i / 8) + 8 g + i % 8: the 8 scores of one 16-key step are the P^T operand.

Software pipeline (one wave per SIMD, so a wave hides its own softmax): phase p issues the MFMAs
of P.V(p-1) and S(p+1) and, between them, the softmax VALU work of half-tile p. Tiles of 64 keys
(two half-tiles) go straight from memory into LDS (buffer_load ... lds) in three stages; the
transfer of tile j+2 is issued at the start of iteration j and waited for at its end, where one
barrier per tile publishes it and frees the stage of tile j-1.

LDS rows are 256 bytes unpadded; the 16-byte chunk c of row r is stored at chunk
c ^ (4 (r & 3) + ((r >> 2) & 3)), which keeps both the row reads (ds_read_b128) and the
transposing reads (ds_read_b64_tr_b16) free of bank conflicts. A transfer instruction fills 1 KiB
(four rows); each lane fetches the global chunk that lands in its swizzled slot.

Memory safety: every global access is a buffer instruction. K/V transfers use a resource bounded
to the live rows of the tile (rows past kv_len read as zeros, masked by the softmax); Q, O and
LSE offsets are formed from clamped row indices, and the stores of rows past the sequence use an
offset beyond the resource range (dropped). All waves of a workgroup run the same tile count, so
every barrier is met by all four waves, and every loop has a trip count fixed at entry.

Hazards: instructions are issued in the order written; the required independent-instruction
distances (MFMA result -> other use 12, VALU write -> MFMA read 2, transcendental -> use 1,
VALU write -> v_permlane32_swap 2, M0 write -> LDS transfer 1) are enforced by a checker that
inserts s_nop over every control-flow path into each block.
"""

from __future__ import annotations

import re
import sys

# --------------------------------------------------------------------------- kernel arguments
# (name, byte offset, size); mirrored by the generated header for the host launcher.
ARGS = [
    ("q", 0, 8), ("k", 8, 8), ("v", 16, 8), ("o", 24, 8), ("lse", 32, 8), ("rope", 40, 8),
    ("q_sb", 48, 8), ("k_sb", 56, 8), ("o_sb", 64, 8), ("lse_sb", 72, 8), ("k_sh", 80, 8),
    ("q_sh", 88, 4), ("o_sh", 92, 4), ("lse_sh", 96, 4), ("q_ss", 100, 4), ("o_ss", 104, 4),
    ("k_ss", 108, 4), ("q_len", 112, 4), ("kv_len", 116, 4), ("gshift", 120, 4),
    ("kv_heads", 124, 4), ("causal", 128, 4), ("causal_off", 132, 4), ("rope_q", 136, 4),
    ("q_rope_off", 140, 4), ("c2", 144, 4), ("nqb", 148, 4), ("nb", 152, 4), ("grid", 156, 4),
    ("units", 160, 4), ("fd_units_m", 164, 4), ("fd_units_s", 168, 4), ("batch", 172, 4),
    ("q_nrec", 176, 4), ("o_nrec", 180, 4), ("lse_nrec", 192, 4), ("fd_kvh_m", 196, 4),
    ("fd_kvh_s", 200, 4), ("rope_bytes", 204, 4),
    # paged kernel only: the block tables (bytes 184..191, unused by the contiguous kernel) and
    # their row stride in entries (the slot of k_sb: a page pool has no batch stride)
    ("bt", 184, 8), ("bt_stride", 56, 4),
    # precise kernel only: bytes from the rotated K to its residual (the same layout after it)
    ("klo_off", 184, 8),
]
ARG_BYTES = 208
S_QNREC, S_ONREC, S_LNREC = 52, 53, 56  # (argument registers of q_nrec, o_nrec, lse_nrec)
S_ROUND = 3           # persistent loop: blocks this workgroup has finished
ARG_SGPR0 = 8  # argument dword i lives in s[8 + i]


def arg(name: str, hi: bool = False) -> str:
    for n, off, sz in ARGS:
        if n == name:
            return f"s{ARG_SGPR0 + off // 4 + (1 if hi else 0)}"
    raise KeyError(name)


def arg64(name: str) -> str:
    for n, off, sz in ARGS:
        if n == name:
            assert sz == 8
            return f"s[{ARG_SGPR0 + off // 4}:{ARG_SGPR0 + off // 4 + 1}]"
    raise KeyError(name)


KERNEL_CONTIG = "fa_prefill_a64_bf16"
KERNEL_PAGED = "fa_prefill_a64_paged_bf16"
KERNEL_PREC = "fa_prefill_a64_precise_bf16"
KERNEL_CONTIG_F16 = "fa_prefill_a64_f16"
KERNEL_PAGED_F16 = "fa_prefill_a64_paged_f16"
KERNEL = KERNEL_CONTIG
# Paged K/V (page size 16): transfer instruction i of a tile covers its rows 16 i .. 16 i + 15,
# i.e. exactly one page, read through a buffer resource based at that page. The page ids of
# the next transfers sit in one VGPR (lane = page of the tile range), loaded a pair ahead.
PAGED = False
# Precise scores: K read as its bf16 high part and the residual (a second LDS tile), Q carried
# the same way (residual in AGPRs), three MFMAs per score k-step (hi.hi + lo.hi + hi.lo)
PREC = False


# f16 storage: the same kernels with the f16 MFMA and f16 conversions; the fast path's overflow
# threshold drops to row sums above 2^15 so that every rounded probability stays finite in f16.
F16 = False


def MF() -> str:
    return "v_mfma_f32_32x32x16_f16" if F16 else "v_mfma_f32_32x32x16_bf16"


def CVT() -> str:
    return "v_cvt_pk_f16_f32" if F16 else "v_cvt_pk_bf16_f32"


def unpack(lo: str, hi: str, src: str) -> list:
    """The two 16-bit values packed in src as f32 in lo (low half) and hi (high half)."""
    if F16:
        return [I(f"v_cvt_f32_f16 {lo}, {src}"),
                I(f"v_cvt_f32_f16_sdwa {hi}, {src} dst_sel:DWORD src0_sel:WORD_1")]
    return [I(f"v_lshlrev_b32 {lo}, 16, {src}"), I(f"v_and_b32 {hi}, 0xffff0000, {src}")]


def STAGE_BYTES() -> int:
    """One LDS stage: K (16 KiB), (precise: K residual, 16 KiB), V (16 KiB)."""
    return 49152 if PREC else 32768


def V_REGION() -> int:
    return 32768 if PREC else 16384
NSTAGE = 5            # LDS stages of (K 16 KiB, V 16 KiB): tiles j .. j + NSTAGE - 1 resident
PAIR = True           # one barrier per two iterations (needs NSTAGE = 5)
ISSUE_WEIGHT = {"trans": 2}  # relative issue cost of an instruction kind in the phase scheduler
LDS_BYTES = NSTAGE * 32768
INVALID_OFF = 0x80000000  # beyond every resource range used for stores
O_ROWB = 272          # O staging in LDS: 64 rows of 256 bytes per wave, padded to 272
O_WAVEB = 64 * O_ROWB

# --------------------------------------------------------------------------- registers
# VGPRs
V_TID = 0
V_LANE = 1
SB = [2, 34]          # score buffers: SB[x] + 16 rb .. +15
PB = [66, 82]         # probability buffers: PB[x] + 8 rb + 4 s .. +3
RK = 4                # K operand ring: operands read ahead (4 registers each)
RV = 3                # V^T operand ring
KRING = 98            # RK slots x 4 (up to 4 here; more go to the spare area)
VRING = 114           # RV slots x 4
VKA = 126             # 8 K read addresses (one per k-step)
VVA = 134             # 8 V^T read addresses (mb * 2 + hi)
VTOFF = 142           # 4 transfer offsets
V_M = 146             # running max per row, in exp2 units (m * scale * log2 e)
V_L = 148             # running sum
V_LT = 150            # this half-tile's partial row sums
V_NBV = 152           # 2 temps: new bias value (-m) per row
V_ALPHA = 154
V_LIMB = 156          # causal/tail limit base per rb
V_LIM = 158
V_MX = 160            # 4 temps for the cross-lane max
V_U = 164             # 2 temps
V_NINF = 166
V_TMP = 168           # 8 temps (rescale)
V_QOFF = 176          # Q byte offsets per rb (2)
V_CSOFF = 178         # (cos, sin) row byte offsets per rb (2)
V_OOFF = 180          # O byte offsets per rb (2)
V_LOFF = 182          # LSE byte offsets per rb (2)
V_ROW = 184           # 4 setup temps
NB = 188              # score bias blocks: NB + 16 rb .. +15 all hold -m of the lane's row
V_BIG = 220           # 2^64: a half-tile row sum above it sends the phase to the exact path
V_EPI = 222           # 4 per-lane epilogue addresses (O staging write/read, row-offset permute, chunk)
V_PT = 226            # paged: page ids, lane l = entry l of the loaded block-table range
V_PTOFF = 227         # paged: 4 * lane (byte offset of the lane's block-table entry)
KLRING = 228          # precise kernel: K residual operand ring (RK slots x 4)
NUM_VGPR = 244
# AGPRs
A_O = 0               # O[rb][mb]: a[(rb*4+mb)*16 ..]
A_Q = 128             # Q[rb][ks]: a[128 + (rb*8+ks)*4 ..]
A_QLO = 192           # precise kernel: the residual of Q, same layout
NUM_AGPR = 192

# SGPRs (beyond s[0:1] kernarg pointer, s2 workgroup id, s[8:59] arguments)
S_WAVE = 60
S_BH = 61
S_QB = 62
S_B = 63
S_KVH = 64
S_N = 65              # tiles of the block
S_NFULL = 66
S_J = 67
S_JU = 68             # end of the unmasked loop
S_NM1 = 69            # n - 1
S_MV = 70             # [70:71] overflow flags of the phase
S_NEED0 = 72          # [72:73]
S_NEED1 = 74          # [74:75]
S_HIMASK = 76         # [76:77] lanes 32..63
S_KEY0 = 78           # first key of the masked half-tile
S_RK = 80             # [80:83] K transfer resource
S_RV = 84             # [84:87] V transfer resource
S_KBASE = 88          # [88:89]
S_VBASE = 90          # [90:91]
S_NREC = 92
S_TSLOT = 93          # stage of the next transfer
S_TT = 94             # tile of the next transfer
S_KDELTA = 95
S_T0 = 96             # [96:99] temps (4-aligned: also a resource)
S_T1 = 97
S_T2 = 98
S_T3 = 99
S_KSLOT = 100
S_VSLOT = 101
S_RQ = 4              # [4:7] Q / O / LSE resource (reused)
NUM_SGPR = 102


def vr(base: int, n: int = 1) -> str:
    return f"v{base}" if n == 1 else f"v[{base}:{base + n - 1}]"


def ar(base: int, n: int = 1) -> str:
    return f"a{base}" if n == 1 else f"a[{base}:{base + n - 1}]"


def sr(base: int, n: int = 1) -> str:
    return f"s{base}" if n == 1 else f"s[{base}:{base + n - 1}]"


def s_of(x: int) -> int:  # score register: buffer x, block rb, value i
    return x


# --------------------------------------------------------------------------- instructions
_REG_RE = re.compile(r"\b([vas])\[(\d+):(\d+)\]|\b([vas])(\d+)\b")


def regs_in(text: str) -> list[str]:
    out = []
    for m in _REG_RE.finditer(text):
        if m.group(1):
            k, a, b = m.group(1), int(m.group(2)), int(m.group(3))
            out += [f"{k}{i}" for i in range(a, b + 1)]
        else:
            out.append(f"{m.group(4)}{m.group(5)}")
    return out


TRANS = ("v_exp_f32", "v_log_f32", "v_rcp_f32")


class Ins:
    __slots__ = ("text", "kind", "reads", "writes", "nops", "dsid", "needs", "srcc_chain")

    def __init__(self, text, kind=None, reads=None, writes=None):
        self.text = text
        op = text.split()[0] if text.strip() else ""
        if kind is None:
            if op.startswith("v_mfma"):
                kind = "mfma"
            elif op.startswith(TRANS):
                kind = "trans"
            elif op.startswith("v_permlane"):
                kind = "permlane"
            elif op.startswith("v_"):
                kind = "valu"
            elif op.startswith("ds_"):
                kind = "ds"
            elif op.startswith("buffer_"):
                kind = "vmem"
            elif op == "s_nop":
                kind = "nop"
            elif op.endswith(":") or op == "":
                kind = "label"
            elif op.startswith("s_"):
                kind = "salu"
            else:
                kind = "other"
        self.kind = kind
        self.nops = 0
        self.dsid = None
        self.needs = []
        self.srcc_chain = False
        if reads is None or writes is None:
            r, w = self._operands()
            reads = r if reads is None else reads
            writes = w if writes is None else writes
        self.reads = set(reads)
        self.writes = set(writes)

    def _operands(self):
        t = self.text.split(None, 1)
        if len(t) < 2:
            return [], []
        op, rest = t
        parts = [p.strip() for p in rest.split(",")]
        if self.kind in ("vmem",):
            if op.startswith("buffer_store"):
                return regs_in(rest), []
            if " lds" in rest:
                return regs_in(rest), []
            return regs_in(",".join(parts[1:])), regs_in(parts[0])
        if self.kind == "ds":
            return regs_in(",".join(parts[1:])), regs_in(parts[0])
        if self.kind == "permlane":
            rr = regs_in(rest)
            return rr, rr
        if self.kind == "salu":
            if op.startswith(("s_cmp", "s_bitcmp", "s_waitcnt", "s_barrier", "s_cbranch",
                              "s_branch", "s_endpgm")):
                return regs_in(rest), []
            return regs_in(",".join(parts[1:])), regs_in(parts[0])
        if op.startswith("v_cmp"):
            return regs_in(",".join(parts[1:])), regs_in(parts[0])
        if op.startswith("v_dot2c"):
            rr = regs_in(rest)
            return rr, regs_in(parts[0])
        return regs_in(",".join(parts[1:])), regs_in(parts[0])

    def ws(self) -> int:
        if self.kind == "label":
            return 0
        if self.kind == "nop":
            return int(self.text.split()[1]) + 1
        return 1


def I(text, **kw) -> Ins:
    return Ins(text, **kw)


# --------------------------------------------------------------------------- hazard checker
def _is_vreg(r: str) -> bool:
    return r[0] in "va"


def required(prev: Ins, cur: Ins) -> int:
    """Independent wait states `cur` needs after `prev` (the rules LLVM's hazard recognizer
    applies on gfx950, verified against the compiler's own output)."""
    if cur.kind in ("label", "nop"):
        return 0
    need = 0
    pw = {r for r in prev.writes if _is_vreg(r)}
    if prev.kind == "mfma" and pw:
        touched = (cur.reads | cur.writes) & pw
        if touched:
            if cur.kind == "mfma" and cur.srcc_chain and touched <= cur.writes:
                pass  # same accumulator, back-to-back chain: handled by the hardware
            else:
                need = max(need, 12)
    if prev.kind in ("valu", "trans", "permlane") and pw:
        if cur.kind == "mfma" and ((cur.reads | cur.writes) & pw):
            need = max(need, 2)
        if cur.kind == "permlane" and (cur.reads & pw):
            need = max(need, 2)
    if prev.kind == "trans" and pw and cur.kind in ("valu", "trans", "permlane"):
        if cur.reads & pw:
            need = max(need, 1)
    if prev.kind == "permlane" and pw and (cur.reads & pw):
        need = max(need, 2)
    # v_dot* execute outside the VALU pipeline: their result reaches another instruction 3
    # wait states later, except the next v_dot* accumulating onto the same register
    if prev.text.startswith("v_dot") and pw and ((cur.reads | cur.writes) & pw):
        chain = cur.text.startswith("v_dot2c") and cur.writes == pw
        if not chain:
            need = max(need, 3)
    if prev.kind == "salu" and "m0" in prev.text.split(",")[0] and cur.kind == "vmem" and " lds" in cur.text:
        need = max(need, 1)
    return need


def check_path(path: list[Ins], start: int):
    """Raise nops of instructions path[start:] so every hazard against any earlier instruction
    of `path` is covered. Instructions before `start` are context (already fixed)."""
    window = 40
    for i in range(start, len(path)):
        cur = path[i]
        if cur.kind in ("label",):
            continue
        dist = cur.nops if cur.kind != "nop" else 0
        req_extra = 0
        j = i - 1
        d = dist
        while j >= 0 and i - j <= window and d < 13:
            p = path[j]
            r = required(p, cur)
            if r > d:
                req_extra = max(req_extra, r - d)
            d += p.ws() + (p.nops if p.kind != "nop" else 0)
            j -= 1
        if req_extra:
            cur.nops += req_extra


class Block:
    def __init__(self, name: str):
        self.name = name
        self.ins: list[Ins] = []
        self.preds: list["Block"] = []

    def add(self, x):
        if isinstance(x, Ins):
            self.ins.append(x)
        elif isinstance(x, str):
            self.ins.append(I(x))
        else:
            for y in x:
                self.add(y)


def tails(block: Block, need_ws: int = 16, depth: int = 4) -> list[list[Ins]]:
    """All instruction tails (>= need_ws wait states) of the paths entering `block`."""
    if depth == 0 or not block.preds:
        return [[]]
    out = []
    for p in block.preds:
        seq = p.ins
        ws = sum(x.ws() + (x.nops if x.kind != "nop" else 0) for x in seq)
        if ws >= need_ws:
            out.append(seq[-40:])
        else:
            for t in tails(p, need_ws - ws, depth - 1):
                out.append(t + seq)
    return out


def fix_hazards(blocks: list[Block]):
    for _ in range(3):  # nops only ever grow; repeat so predecessors' nops are counted
        for b in blocks:
            for t in tails(b):
                check_path(t + b.ins, len(t))


# --------------------------------------------------------------------------- helpers
def valu(text):
    return I(text)


def fdiv(dst, n, m, s, tmp):
    """dst = n / d for the FastDiv magic (m, s) of d: (mulhi(n, m) + n) >> s (n < 2^24)."""
    return [I(f"s_mul_hi_u32 {tmp}, {n}, {m}"), I(f"s_add_u32 {tmp}, {tmp}, {n}"),
            I(f"s_lshr_b32 {dst}, {tmp}, {s}")]


def swz_py(r: int) -> int:
    return 4 * (r & 3) + ((r >> 2) & 3)


# --------------------------------------------------------------------------- the program
class Gen:
    def __init__(self):
        self.blocks: list[Block] = []
        self.cur: Block | None = None
        self.ds_outstanding: list[int] = []  # ids of LDS reads in flight (oldest first)
        self.ds_next = 0

    def new_block(self, name, preds=()):
        b = Block(name)
        b.preds = list(preds)
        self.blocks.append(b)
        self.cur = b
        return b

    def emit(self, x):
        self.cur.add(x)

    # ---- LDS read bookkeeping (in-order completion: lgkmcnt counts younger reads)
    def ds_issue(self, text) -> int:
        ins = I(text)
        ins.dsid = self.ds_next
        self.ds_next += 1
        self.ds_outstanding.append(ins.dsid)
        self.emit(ins)
        return ins.dsid

    def ds_wait_for(self, ids):
        if not ids:
            return
        pend = [i for i in ids if i in self.ds_outstanding]
        if not pend:
            return
        last = max(self.ds_outstanding.index(i) for i in pend)
        younger = len(self.ds_outstanding) - 1 - last
        n = min(younger, 15)
        self.emit(I(f"s_waitcnt lgkmcnt({n})"))
        self.ds_outstanding = self.ds_outstanding[len(self.ds_outstanding) - n:] if n else []

    def ds_wait_all(self):
        if self.ds_outstanding:
            self.emit(I("s_waitcnt lgkmcnt(0)"))
            self.ds_outstanding = []


# ---- operand reads ----------------------------------------------------------------------------
def k_read_text(slot: int, ks: int, hh: int) -> str:
    return f"ds_read_b128 {vr(KRING + 4 * slot, 4)}, {vr(VKA + ks)} offset:{hh * 8192}"


def klo_read_text(slot: int, ks: int, hh: int) -> str:
    """Precise kernel: the K residual operand (second tile of the stage)."""
    return f"ds_read_b128 {vr(KLRING + 4 * slot, 4)}, {vr(VKA + ks)} offset:{16384 + hh * 8192}"


def q_lo_op(rb: int, ks: int) -> str:
    return ar(A_QLO + (rb * 8 + ks) * 4, 4)


def s_parts() -> list:
    """(K ring, Q operand function) of the score MFMAs of one k-step: one, or three (precise)."""
    if not PREC:
        return [(KRING, q_op)]
    return [(KRING, q_op), (KLRING, q_op), (KRING, q_lo_op)]


def v_read_texts(slot: int, mb: int, s: int, hh: int) -> list[str]:
    off = hh * 8192 + s * 4096
    base = VRING + 4 * slot
    return [f"ds_read_b64_tr_b16 {vr(base, 2)}, {vr(VVA + mb * 2 + 0)} offset:{off}",
            f"ds_read_b64_tr_b16 {vr(base + 2, 2)}, {vr(VVA + mb * 2 + 1)} offset:{off}"]


def q_op(rb: int, ks: int) -> str:
    return ar(A_Q + (rb * 8 + ks) * 4, 4)


def o_acc(rb: int, mb: int) -> str:
    return ar(A_O + (rb * 4 + mb) * 16, 16)


def s_acc(x: int, rb: int) -> str:
    return vr(SB[x] + 16 * rb, 16)


def p_op(x: int, rb: int, s: int) -> str:
    return vr(PB[x] + 8 * rb + 4 * s, 4)


# ---- softmax VALU program of one half-tile --------------------------------------------------
# Scores arrive as S' = S * c2 - m (the first MFMA of a score block accumulates onto the bias
# block NB = -m, and Q carries the factor c2 = scale * log2 e), so P = exp2(S') needs one
# instruction per score. The running max m is not recomputed per tile: a half-tile whose row sum
# exceeds 2^64 (an exponent that would overflow, or the first tile, taken exactly by the
# prologue) sends the phase to the exact path, which recomputes that half-tile's scores, takes
# the row maxima, moves m, rescales O and l and redoes P. With m at least the first half-tile's
# row max, every row keeps l >= 1 and P stays below 2^64, so O and l cannot overflow in f32.
def mask_program(x: int) -> list[Ins]:
    out = []
    S = SB[x]
    for rb in range(2):
        out.append(I(f"v_subrev_u32 {vr(V_LIM + rb)}, {sr(S_KEY0)}, {vr(V_LIMB + rb)}"))
    for rb in range(2):
        for i in range(16):
            key = 16 * (i >> 3) + (i & 7)
            out.append(I(f"v_cmp_gt_i32 vcc, {key}, {vr(V_LIM + rb)}",
                         reads=[f"v{V_LIM + rb}"], writes=["vcc"]))
            reg = S + 16 * rb + i
            out.append(I(f"v_cndmask_b32 {vr(reg)}, {vr(reg)}, {vr(V_NINF)}, vcc",
                         reads=[f"v{reg}", f"v{V_NINF}", "vcc"], writes=[f"v{reg}"]))
    return out


def exp_pack_sum(x: int) -> list[Ins]:
    """P^T = bf16(exp2(S')) into PB[x] and the half-tile row sums of P into V_LT: f32 sums of the
    rounded probabilities the P.V product uses (so O = sum p v / sum p stays a convex combination
    of V rows; the stale running max leaves the dominant p off a power of two, where summing the
    unrounded values would bias O by up to 2^-9 relative). The rounded halves are unpacked into
    the exponentials' registers (a shift and an and): v_dot* instructions would sum the packed
    pairs directly but issue to the matrix pipeline and stall behind the MFMAs."""
    out = []
    S = SB[x]
    pend = []
    for rb in range(2):
        for s in range(2):
            for j in range(4):
                i0 = 8 * s + 2 * j
                r = S + 16 * rb + i0
                out += [I(f"v_exp_f32 {vr(r)}, {vr(r)}"), I(f"v_exp_f32 {vr(r + 1)}, {vr(r + 1)}")]
                out += pend
                pend = []
                dst = PB[x] + 8 * rb + 4 * s + j
                pend += [I(f"{CVT()} {vr(dst)}, {vr(r)}, {vr(r + 1)}")] + \
                    unpack(vr(r), vr(r + 1), vr(dst))
                lt = vr(V_LT + rb)
                if i0 == 0:
                    pend.append(I(f"v_add_f32 {lt}, {vr(r)}, {vr(r + 1)}"))
                else:
                    pend += [I(f"v_add_f32 {lt}, {lt}, {vr(r)}"),
                             I(f"v_add_f32 {lt}, {lt}, {vr(r + 1)}")]
    out += pend
    return out


def softmax_program(x: int, masked: bool) -> list[Ins]:
    """Fast path of the half-tile in SB[x]: (mask,) exponentials, P^T, row sums, overflow flags."""
    out = mask_program(x) if masked else []
    out += exp_pack_sum(x)
    out += [I(f"v_cmp_gt_f32 {sr(S_NEED0, 2)}, {vr(V_LT)}, {vr(V_BIG)}",
              reads=[f"v{V_LT}", f"v{V_BIG}"], writes=[f"s{S_NEED0}", f"s{S_NEED0 + 1}"]),
            I(f"v_cmp_gt_f32 {sr(S_NEED1, 2)}, {vr(V_LT + 1)}, {vr(V_BIG)}",
              reads=[f"v{V_LT + 1}", f"v{V_BIG}"], writes=[f"s{S_NEED1}", f"s{S_NEED1 + 1}"]),
            I(f"s_or_b64 {sr(S_MV, 2)}, {sr(S_NEED0, 2)}, {sr(S_NEED1, 2)}")]
    return out


def rescale_block() -> list[Ins]:
    """O^T *= alpha (per row)."""
    out = []
    for rb in range(2):
        for mb in range(4):
            base = A_O + (rb * 4 + mb) * 16
            for h in range(2):
                regs = [base + 8 * h + i for i in range(8)]
                out += [I(f"v_accvgpr_read_b32 {vr(V_TMP + i)}, {ar(a)}") for i, a in enumerate(regs)]
                out += [I(f"v_mul_f32 {vr(V_TMP + i)}, {vr(V_TMP + i)}, {vr(V_ALPHA + rb)}")
                        for i in range(8)]
                out += [I(f"v_accvgpr_write_b32 {ar(a)}, {vr(V_TMP + i)}") for i, a in enumerate(regs)]
    return out


def exact_path(gen: "Gen", x: int, hh: int, s_x) -> None:
    """Exact softmax of the half-tile whose scores belong in SB[x] (K half hh of the stage before
    the current K read stage): recompute the raw scores S * c2, mask, take the row maxima, move m
    (alpha = exp2(m_old - m_new)), rescale O and l, re-bias the scores SB[s_x] that this phase's
    MFMAs accumulated onto the old bias, set the bias blocks, and redo P^T and the row sums."""
    e = gen.emit
    gen.ds_wait_all()
    e(I("s_waitcnt lgkmcnt(0)"))
    _recompute_scores(gen, x, hh)
    e(mask_program(x))
    _exact_softmax(gen, x, s_x)


def _recompute_scores(gen: "Gen", x: int, hh: int) -> None:
    """SB[x] = the raw scores S * c2 of K half hh of the stage before the current K stage."""
    e = gen.emit
    # K addresses of the previous stage
    d = sr(S_T0)
    e([I(f"s_cmp_eq_u32 {sr(S_KSLOT)}, 0"),
       I(f"s_mov_b32 {d}, 0x{(-STAGE_BYTES()) & 0xffffffff:x}"),
       I(f"s_cselect_b32 {d}, 0x{(NSTAGE - 1) * STAGE_BYTES():x}, {d}")])
    e([I(f"v_add_u32 {vr(V_TMP + i)}, {d}, {vr(VKA + i)}") for i in range(8)])
    for half in range(2):
        for k4 in range(4):
            ks = 4 * half + k4
            e(I(f"ds_read_b128 {vr(KRING + 4 * k4, 4)}, {vr(V_TMP + ks)} offset:{hh * 8192}"))
            if PREC:
                e(I(f"ds_read_b128 {vr(KLRING + 4 * k4, 4)}, {vr(V_TMP + ks)} "
                    f"offset:{16384 + hh * 8192}"))
        e(I("s_waitcnt lgkmcnt(0)"))
        for k4 in range(4):
            ks = 4 * half + k4
            for part, (ring, qf) in enumerate(s_parts()):
                for rb in range(2):
                    src_c = "0" if ks == 0 and part == 0 else s_acc(x, rb)
                    ins = I(f"{MF()} {s_acc(x, rb)}, {vr(ring + 4 * k4, 4)}, "
                            f"{qf(rb, ks)}, {src_c}")
                    ins.srcc_chain = not (ks == 0 and part == 0)
                    e(ins)


def _row_max(gen: "Gen", x: int):
    """Both 32-row blocks' maxima of the masked raw scores in SB[x], on every lane: returns the
    registers holding block 0's and block 1's."""
    e = gen.emit
    S = SB[x]
    for rb in range(2):
        r = S + 16 * rb
        t = V_MX + 2 * rb
        e([I(f"v_max3_f32 {vr(t)}, {vr(r)}, {vr(r + 1)}, {vr(r + 2)}"),
           I(f"v_max3_f32 {vr(t + 1)}, {vr(r + 3)}, {vr(r + 4)}, {vr(r + 5)}"),
           I(f"v_max3_f32 {vr(t)}, {vr(t)}, {vr(r + 6)}, {vr(r + 7)}"),
           I(f"v_max3_f32 {vr(t + 1)}, {vr(t + 1)}, {vr(r + 8)}, {vr(r + 9)}"),
           I(f"v_max3_f32 {vr(t)}, {vr(t)}, {vr(r + 10)}, {vr(r + 11)}"),
           I(f"v_max3_f32 {vr(t + 1)}, {vr(t + 1)}, {vr(r + 12)}, {vr(r + 13)}"),
           I(f"v_max3_f32 {vr(t)}, {vr(t)}, {vr(r + 14)}, {vr(r + 15)}")])
    mx0, mx1 = V_U, V_U + 1
    F, G = V_MX, V_MX + 1
    # swap(mx0.hi, mx1.lo): max(mx0, mx1) is row 0's max on lanes < 32 and row 1's on lanes >= 32;
    # a second swap of that value against its copy gives both rows' maxima on every lane
    e([I(f"v_max_f32 {vr(mx0)}, {vr(V_MX)}, {vr(V_MX + 1)}"),
       I(f"v_max_f32 {vr(mx1)}, {vr(V_MX + 2)}, {vr(V_MX + 3)}"),
       I(f"v_permlane32_swap_b32 {vr(mx0)}, {vr(mx1)}"),
       I(f"v_max_f32 {vr(F)}, {vr(mx0)}, {vr(mx1)}"),
       I(f"v_mov_b32 {vr(G)}, {vr(F)}"),
       I(f"v_permlane32_swap_b32 {vr(F)}, {vr(G)}")])
    return F, G


def first_max(gen: "Gen", x: int) -> None:
    """The block's first half-tile (raw scores in SB[x], masked): m = its row maxima, the bias
    blocks -m for the next scores, SB[x] biased to S' = S * c2 - m. O and l are still zero."""
    e = gen.emit
    F, G = _row_max(gen, x)
    for rb, mt in ((0, F), (1, G)):
        e([I(f"v_mov_b32 {vr(V_M + rb)}, {vr(mt)}"),
           I(f"v_xor_b32 {vr(V_NBV + rb)}, 0x80000000, {vr(mt)}")])
    for rb in range(2):
        e([I(f"v_mov_b32 {vr(NB + 16 * rb + i)}, {vr(V_NBV + rb)}") for i in range(16)])
        r = SB[x] + 16 * rb
        e([I(f"v_add_f32 {vr(r + i)}, {vr(r + i)}, {vr(V_NBV + rb)}") for i in range(16)])


def _exact_softmax(gen: "Gen", x: int, s_x) -> None:
    """Row maxima of the masked raw scores in SB[x], the move of m, rescale, re-bias, redo P."""
    e = gen.emit
    S = SB[x]
    F, G = _row_max(gen, x)
    for rb, mt in ((0, F), (1, G)):
        m, al, nbv = V_M + rb, V_ALPHA + rb, V_NBV + rb
        e([I(f"v_max_f32 {vr(mt)}, {vr(mt)}, {vr(m)}"),            # m_new (finite)
           I(f"v_sub_f32 {vr(al)}, {vr(m)}, {vr(mt)}"),
           I(f"v_exp_f32 {vr(al)}, {vr(al)}"),                      # m_old = -inf: 0
           I(f"v_mov_b32 {vr(m)}, {vr(mt)}"),
           I(f"v_mul_f32 {vr(V_L + rb)}, {vr(V_L + rb)}, {vr(al)}"),
           I(f"v_xor_b32 {vr(nbv)}, 0x80000000, {vr(mt)}"),        # new bias -m_new
           I(f"v_sub_f32 {vr(V_U + rb)}, {vr(nbv)}, {vr(NB + 16 * rb)}")])  # bias change
    if s_x is not None:
        for rb in range(2):
            r = SB[s_x] + 16 * rb
            e([I(f"v_add_f32 {vr(r + i)}, {vr(r + i)}, {vr(V_U + rb)}") for i in range(16)])
    for rb in range(2):
        e([I(f"v_mov_b32 {vr(NB + 16 * rb + i)}, {vr(V_NBV + rb)}") for i in range(16)])
    e(rescale_block())
    for rb in range(2):
        r = S + 16 * rb
        e([I(f"v_add_f32 {vr(r + i)}, {vr(r + i)}, {vr(V_NBV + rb)}") for i in range(16)])
    e(exp_pack_sum(x))


# ---- one pipeline phase ------------------------------------------------------------------------
def phase(gen: Gen, *, pv_x, pv_hh, s_x, s_hh, sm_x, sm_masked, pre=(),
          prefetch_v_hh=None, after_last_v=(), after_last_k=(), vring_state=None, spread=(),
          zero_bias=False):
    """Emits one phase: MFMAs of P.V (P in PB[pv_x], V half pv_hh of the current V stage) then
    S (into SB[s_x], K half s_hh), with the softmax of SB[sm_x] spread between them.
    spread: instruction groups (the tile transfers) issued one every few MFMAs from the third
    on, so that the memory pipeline takes them one at a time instead of in a burst.
    zero_bias: the scores' first k-step accumulates onto 0 instead of the bias blocks.
    vring_state: dict carrying the V operands already read into the ring by the previous phase:
    {'ready': {op_index: (slot, [ds ids])}}, and after the phase the prefetched operands of the
    next phase. Returns the new ring state."""
    mf: list[tuple[str, list, dict]] = []  # (text, operand key, info)
    # P.V: operand o = (s, mb) in order s-major; each operand feeds rb = 0, 1
    pv_ops = [(s, mb) for s in range(2) for mb in range(4)] if pv_x is not None else []
    k_ops = list(range(8)) if s_x is not None else []
    DV, DK = RV, RK
    ready = dict(vring_state["ready"]) if vring_state else {}
    # slots: V ring slots 0..2; op o uses slot o % 3 (ready ops from the previous phase agree)
    valu_stream = softmax_program(sm_x, sm_masked) if sm_x is not None else []
    # the phase's scalar set-up (transfers, key base) is spread over the first MFMA slots
    valu_stream = list(pre) + valu_stream
    # plan MFMA list
    mlist = []
    for oi, (s, mb) in enumerate(pv_ops):
        for rb in range(2):
            mlist.append(("pv", oi, rb))
    for ks in k_ops:
        for part in range(len(s_parts())):
            for rb in (0, 1):
                mlist.append(("s", ks, rb, part))
    nm = len(mlist)
    vi = 0  # next VALU item

    # issue helpers
    v_issued = {}   # op index -> ds ids
    k_issued = {}
    v_slot_free_after = {}  # slot -> index in mlist of last MFMA using it (must be issued)
    for oi, ids in ready.items():
        v_issued[oi] = ids
    next_v = max(ready.keys()) + 1 if ready else 0
    next_k = 0
    issued_m = -1  # index of last MFMA emitted

    def v_slot(oi):
        return oi % DV

    def last_use_v(oi):  # mlist index of the last MFMA reading operand oi
        return 2 * oi + 1

    last_k = {}
    for i_, m_ in enumerate(mlist):
        if m_[0] == "s":
            last_k[m_[1]] = i_

    def last_use_k(ks):
        return last_k[ks]

    def can_issue_v(oi):
        prev = oi - DV
        return prev < 0 or last_use_v(prev) <= issued_m

    def can_issue_k(ks):
        prev = ks - DK
        return prev < 0 or last_use_k(prev) <= issued_m

    def issue_reads(budget):
        nonlocal next_v, next_k
        n = 0
        while n < budget:
            if next_v < len(pv_ops) and can_issue_v(next_v):
                s, mb = pv_ops[next_v]
                ids = [gen.ds_issue(t) for t in v_read_texts(v_slot(next_v), mb, s, pv_hh)]
                v_issued[next_v] = ids
                if next_v == len(pv_ops) - 1:
                    for x in after_last_v:
                        gen.emit(x)
                next_v += 1
                n += 1
                continue
            if next_k < len(k_ops) and can_issue_k(next_k):
                k_issued[next_k] = [gen.ds_issue(k_read_text(next_k % DK, next_k, s_hh))]
                if PREC:
                    k_issued[next_k].append(
                        gen.ds_issue(klo_read_text(next_k % DK, next_k, s_hh)))
                if next_k == len(k_ops) - 1:
                    for x in after_last_k:
                        gen.emit(x)
                next_k += 1
                n += 1
                continue
            break
        return n

    spread = list(spread)
    sp_stride = max(1, min(3, (nm - 4) // max(1, len(spread))))
    n_pre = len(pre)
    next_sp = 2
    # initial reads: fill the rings
    issue_reads(DV + DK)
    total_valu = len(valu_stream)
    # issue cost of the stream: a transcendental takes about twice an ordinary VALU slot
    cost = [ISSUE_WEIGHT.get(x.kind, 1) for x in valu_stream]
    left = sum(cost)
    for mi, m_ in enumerate(mlist):
        kind, idx, rb = m_[:3]
        if kind == "pv":
            gen.ds_wait_for(v_issued[idx])
            s, mb = pv_ops[idx]
            slot = v_slot(idx)
            ins = I(f"{MF()} {o_acc(rb, mb)}, {vr(VRING + 4 * slot, 4)}, "
                    f"{p_op(pv_x, rb, s)}, {o_acc(rb, mb)}")
            ins.srcc_chain = True
        else:
            part = m_[3]
            ring, qf = s_parts()[part]
            gen.ds_wait_for(k_issued[idx])
            slot = idx % DK
            # k-step 0 accumulates onto the bias block (-m of the lane's row)
            first = idx == 0 and part == 0
            src_c = ("0" if zero_bias else vr(NB + 16 * rb, 16)) if first else s_acc(s_x, rb)
            ins = I(f"{MF()} {s_acc(s_x, rb)}, {vr(ring + 4 * slot, 4)}, "
                    f"{qf(rb, idx)}, {src_c}")
            ins.srcc_chain = not first
        gen.emit(ins)
        issued_m = mi
        # (a group needs the scalar set-up of `pre`, which the VALU stream emits first)
        if spread and mi >= next_sp and vi >= n_pre:
            gen.emit(spread.pop(0))
            next_sp = mi + sp_stride
        issue_reads(2)
        # spread the VALU work evenly (by issue cost) over the remaining MFMAs
        remaining_m = nm - mi
        budget = (left + remaining_m - 1) // remaining_m if remaining_m else 0
        spent = 0
        while vi < total_valu and spent < budget:
            gen.emit(valu_stream[vi])
            spent += cost[vi]
            left -= cost[vi]
            vi += 1
    while vi < total_valu:
        gen.emit(valu_stream[vi])
        vi += 1
    for g in spread:
        gen.emit(g)
    issue_reads(99)
    # prefetch the next phase's first V operands
    new_ready = {}
    if prefetch_v_hh is not None:
        s_h = prefetch_v_hh
        for oi in range(DV):
            s, mb = (oi // 4, oi % 4)
            ids = [gen.ds_issue(t) for t in v_read_texts(oi % DV, mb, s, s_h)]
            new_ready[oi] = (oi % DV, ids)
    return {"ready": {k: v[1] for k, v in new_ready.items()}} if new_ready else None


def transfer_block(which: str) -> list[Ins]:
    """The 4 K or V transfer instructions of this wave for the tile whose resource is set up:
    instruction i fills KiB 4 wave + i of the region (rows 16 wave + 4 i .. + 3). One M0 = stage
    base (S_T2, which includes the wave's 4 KiB) + region serves all four: the instruction offset
    1024 i moves the LDS and the global address alike, and the lane offsets VTOFF + i carry
    -1024 i."""
    out = []
    rs = S_RV if which == "v" else S_RK
    region = {"k": 0, "klo": 16384, "v": V_REGION()}[which]
    if which == "klo":
        # the K resource moved to the residual copy (the same rows klo_off bytes further)
        out += [I(f"s_add_u32 {sr(S_RK)}, {sr(S_RK)}, {arg('klo_off')}"),
                I(f"s_addc_u32 {sr(S_RK + 1)}, {sr(S_RK + 1)}, {arg('klo_off', True)}"),
                I(f"s_and_b32 {sr(S_RK + 1)}, {sr(S_RK + 1)}, 0xffff")]
    out.append(I(f"s_add_u32 m0, {sr(S_T2)}, {region}", writes=["m0"], reads=[f"s{S_T2}"]))
    for i in range(4):
        out.append(I(f"buffer_load_dwordx4 {vr(VTOFF + i)}, {sr(rs, 4)}, 0 offen "
                     f"offset:{1024 * i} lds"))
    return out


def kv_transfers() -> list[Ins]:
    """The wave's K (and, precise, K residual) and V transfer instructions of the tile whose
    resources transfer_setup built."""
    return (transfer_block("k") + (transfer_block("klo") if PREC else []) +
            transfer_block("v"))


def transfer_setup(tile_sgpr: str) -> list[Ins]:
    """Resources of the K and V rows of tile `tile_sgpr` (bounded to its live rows) and the
    stage base S_T2 = stage * stage bytes + 4 wave KiB."""
    t0, t1 = sr(S_T0), sr(S_T1)
    rb = arg("k_ss")
    out = [
        # byte offset of the tile: tile * 64 * row_bytes
        I(f"s_mul_i32 {t0}, {tile_sgpr}, {rb}"),
        I(f"s_lshl_b32 {t0}, {t0}, 6"),
        I(f"s_sub_u32 {t1}, {sr(S_NREC)}, {t0}"),
        I(f"s_cmp_lt_i32 {t1}, 0"),
        I(f"s_cselect_b32 {t1}, 0, {t1}"),
        I(f"s_cmp_lt_i32 {tile_sgpr}, {sr(S_N)}"),
        I(f"s_cselect_b32 {t1}, {t1}, 0"),
        I(f"s_add_u32 {sr(S_RK)}, {sr(S_KBASE)}, {t0}"),
        I(f"s_addc_u32 {sr(S_RK + 1)}, {sr(S_KBASE + 1)}, 0"),
        I(f"s_and_b32 {sr(S_RK + 1)}, {sr(S_RK + 1)}, 0xffff"),
        I(f"s_mov_b32 {sr(S_RK + 2)}, {t1}"),
        I(f"s_mov_b32 {sr(S_RK + 3)}, 0x20000"),
        I(f"s_add_u32 {sr(S_RV)}, {sr(S_VBASE)}, {t0}"),
        I(f"s_addc_u32 {sr(S_RV + 1)}, {sr(S_VBASE + 1)}, 0"),
        I(f"s_and_b32 {sr(S_RV + 1)}, {sr(S_RV + 1)}, 0xffff"),
        I(f"s_mov_b32 {sr(S_RV + 2)}, {t1}"),
        I(f"s_mov_b32 {sr(S_RV + 3)}, 0x20000"),
        # stage base: tslot * stage bytes + wave KiB
        (I(f"s_mul_i32 {sr(S_T2)}, {sr(S_TSLOT)}, {STAGE_BYTES()}") if PREC else
         I(f"s_lshl_b32 {sr(S_T2)}, {sr(S_TSLOT)}, 15")),
        I(f"s_lshl_b32 {sr(S_T3)}, {sr(S_WAVE)}, 12"),
        I(f"s_add_u32 {sr(S_T2)}, {sr(S_T2)}, {sr(S_T3)}"),
    ]
    return out


S_PLO = 92            # paged: temps of the page offset (S_NREC is unused there) and
S_PHI = 23            # argument dword 15 (the upper half of the k_sb slot, unused when paged)


def transfer_paged(tile_sgpr: str, lane_base: int) -> list[Ins]:
    """Paged: the wave's 8 transfers of tile `tile_sgpr` into stage S_TSLOT. A wave's four K (and
    four V) instructions cover rows 16 wave .. 16 wave + 15 of the tile, i.e. exactly page `wave`
    of the tile (one page of 16 rows), whose id is V_PT lane lane_base + wave: one buffer
    resource based at that page of this kv head, bounded to the page's live rows (0 past
    kv_len), and one M0 per K or V block (instruction offsets 1024 i, the in-page lane offsets
    VTOFF + i carrying -1024 i)."""
    T0, T1, T2, T3 = (sr(S_T0), sr(S_T1), sr(S_T2), sr(S_T3))
    LO, HI = sr(S_PLO), sr(S_PHI)
    rbytes = arg("k_ss")
    out = [I(f"s_lshl_b32 {T0}, {tile_sgpr}, 6"),                # key of the tile's page 0
           I(f"s_lshl_b32 {T3}, {sr(S_WAVE)}, 4"),
           I(f"s_add_u32 {T0}, {T0}, {T3}"),                       # key of the wave's page
           I(f"s_add_u32 {T1}, {sr(S_WAVE)}, {lane_base}"),
           I(f"v_readlane_b32 {T1}, {vr(V_PT)}, {T1}"),            # page id
           I(f"s_sub_u32 {T3}, {arg('kv_len')}, {T0}"),
           I(f"s_max_i32 {T3}, {T3}, 0"),
           I(f"s_min_i32 {T3}, {T3}, 16"),
           I(f"s_mul_i32 {T3}, {T3}, {rbytes}"),                   # live bytes of the page
           I(f"s_lshl_b32 {LO}, {rbytes}, 4"),                     # page bytes
           I(f"s_mul_hi_u32 {HI}, {T1}, {LO}"),
           I(f"s_mul_i32 {LO}, {T1}, {LO}"),                       # page * page bytes (64-bit)
           I(f"s_add_u32 {sr(S_RK)}, {sr(S_KBASE)}, {LO}"),
           I(f"s_addc_u32 {sr(S_RK + 1)}, {sr(S_KBASE + 1)}, {HI}"),
           I(f"s_and_b32 {sr(S_RK + 1)}, {sr(S_RK + 1)}, 0xffff"),
           I(f"s_mov_b32 {sr(S_RK + 2)}, {T3}"),
           I(f"s_mov_b32 {sr(S_RK + 3)}, 0x20000"),
           I(f"s_add_u32 {sr(S_RV)}, {sr(S_VBASE)}, {LO}"),
           I(f"s_addc_u32 {sr(S_RV + 1)}, {sr(S_VBASE + 1)}, {HI}"),
           I(f"s_and_b32 {sr(S_RV + 1)}, {sr(S_RV + 1)}, 0xffff"),
           I(f"s_mov_b32 {sr(S_RV + 2)}, {T3}"),
           I(f"s_mov_b32 {sr(S_RV + 3)}, 0x20000"),
           I(f"s_lshl_b32 {T2}, {sr(S_TSLOT)}, 15"),
           I(f"s_lshl_b32 {T3}, {sr(S_WAVE)}, 12"),
           I(f"s_add_u32 {T2}, {T2}, {T3}")]                       # stage base + 4 wave KiB
    return out + paged_loads()


def paged_loads() -> list[Ins]:
    """The wave's 8 transfer instructions of the tile whose page resources transfer_paged set."""
    out = []
    for region, rs in ((0, S_RK), (16384, S_RV)):
        out.append(I(f"s_add_u32 m0, {sr(S_T2)}, {region}", writes=["m0"], reads=[f"s{S_T2}"]))
        out += [I(f"buffer_load_dwordx4 {vr(VTOFF + i)}, {sr(rs, 4)}, 0 offen "
                  f"offset:{1024 * i} lds") for i in range(4)]
    return out


def pt_load(first_tile_sgpr: str) -> list[Ins]:
    """Paged: V_PT lane l = block-table entry 4 * first_tile + l of this block's sequence (the
    resource in S_RQ spans its row; entries past it read 0, only used with zero-length pages)."""
    T0 = sr(S_T0)
    return [I(f"s_lshl_b32 {T0}, {first_tile_sgpr}, 4"),
            I(f"buffer_load_dword {vr(V_PT)}, {vr(V_PTOFF)}, {sr(S_RQ, 4)}, {T0} offen")]


def bt_resource() -> list[Ins]:
    """Paged: S_RQ = the block-table row of sequence S_B (bt_stride entries)."""
    T0 = sr(S_T0)
    return [I(f"s_mul_i32 {T0}, {sr(S_B)}, {arg('bt_stride')}"),
            I(f"s_lshl_b32 {T0}, {T0}, 2"),
            I(f"s_add_u32 {sr(S_RQ)}, {arg('bt')}, {T0}"),
            I(f"s_addc_u32 {sr(S_RQ + 1)}, {arg('bt', True)}, 0"),
            I(f"s_and_b32 {sr(S_RQ + 1)}, {sr(S_RQ + 1)}, 0xffff"),
            I(f"s_lshl_b32 {sr(S_RQ + 2)}, {arg('bt_stride')}, 2"),
            I(f"s_mov_b32 {sr(S_RQ + 3)}, 0x20000")]


def advance_slot(slot_sgpr: int, addr_base: int, n_addr: int) -> list[Ins]:
    """slot = (slot + 1) % NSTAGE and every read address += the matching stage delta."""
    d = sr(S_KDELTA)
    s = sr(slot_sgpr)
    out = [I(f"s_add_u32 {s}, {s}, 1"),
           I(f"s_cmp_eq_u32 {s}, {NSTAGE}"),
           I(f"s_cselect_b32 {s}, 0, {s}"),
           I(f"s_mov_b32 {d}, 0x{STAGE_BYTES():x}"),
           I(f"s_cselect_b32 {d}, 0x{(-(NSTAGE - 1) * STAGE_BYTES()) & 0xffffffff:x}, {d}")]
    out += [I(f"v_add_u32 {vr(addr_base + i)}, {d}, {vr(addr_base + i)}") for i in range(n_addr)]
    return out


# --------------------------------------------------------------------------- setup code
def setup(gen: Gen):
    e = gen.emit
    e(I("s_load_dwordx16 s[8:23], s[0:1], 0x0"))
    e(I("s_load_dwordx16 s[24:39], s[0:1], 0x40"))
    e(I("s_load_dwordx16 s[40:55], s[0:1], 0x80"))
    e(I("s_load_dwordx4 s[56:59], s[0:1], 0xc0"))
    e(I(f"v_and_b32 {vr(V_LANE)}, 63, {vr(V_TID)}"))
    e(I(f"v_readfirstlane_b32 {sr(S_WAVE)}, {vr(V_TID)}"))
    e(I("s_waitcnt lgkmcnt(0)"))
    e(I("s_nop 4"))
    e(I(f"s_lshr_b32 {sr(S_WAVE)}, {sr(S_WAVE)}, 6"))
    T0, T1, T2, T3 = (sr(S_T0), sr(S_T1), sr(S_T2), sr(S_T3))
    e([I(f"v_mov_b32 {vr(V_NINF)}, 0xff800000"),
       I(f"v_mov_b32 {vr(V_BIG)}, {'0x47000000' if F16 else '0x5f800000'}"),
       I(f"s_mov_b32 {sr(S_HIMASK)}, 0"),
       I(f"s_mov_b32 {sr(S_HIMASK + 1)}, -1"),
       I(f"s_mov_b32 {sr(S_ROUND)}, 0")])
    # epilogue addresses (constant per lane): O staging write base wave * O_WAVEB +
    # (lane & 31) * O_ROWB + 8 g; read base wave * O_WAVEB + (lane >> 4) * O_ROWB +
    # 16 (lane & 15); row-offset permute source (lane >> 4) * 4; chunk byte 16 (lane & 15)
    e(I(f"v_lshlrev_b32 {vr(V_PTOFF)}, 2, {vr(V_LANE)}"))
    W, R, P, C = V_EPI, V_EPI + 1, V_EPI + 2, V_EPI + 3
    e([I(f"s_mul_i32 {T0}, {sr(S_WAVE)}, {O_WAVEB}"),
       I(f"v_and_b32 {vr(V_TMP)}, 31, {vr(V_LANE)}"),
       I(f"v_mov_b32 {vr(V_TMP + 1)}, {O_ROWB}"),
       I(f"v_mul_u32_u24 {vr(W)}, {vr(V_TMP)}, {vr(V_TMP + 1)}"),
       I(f"v_add_u32 {vr(W)}, {T0}, {vr(W)}"),
       I(f"v_lshrrev_b32 {vr(V_TMP)}, 5, {vr(V_LANE)}"),
       I(f"v_lshl_add_u32 {vr(W)}, {vr(V_TMP)}, 3, {vr(W)}"),
       I(f"v_lshrrev_b32 {vr(V_TMP)}, 4, {vr(V_LANE)}"),
       I(f"v_lshlrev_b32 {vr(P)}, 2, {vr(V_TMP)}"),
       I(f"v_mul_u32_u24 {vr(R)}, {vr(V_TMP)}, {vr(V_TMP + 1)}"),
       I(f"v_add_u32 {vr(R)}, {T0}, {vr(R)}"),
       I(f"v_and_b32 {vr(V_TMP)}, 15, {vr(V_LANE)}"),
       I(f"v_lshlrev_b32 {vr(C)}, 4, {vr(V_TMP)}"),
       I(f"v_add_u32 {vr(R)}, {vr(R)}, {vr(C)}")])


def setup_block(gen: Gen):
    """Per-block set-up of the persistent loop. Blocks are ranked heaviest first (query block
    qb = nqb - 1 - o / units, unit bh = o % units, so every causal rank holds equal work) and dealt
    to the grid's workgroups in snake order: round r gives workgroup w the block
    o = r * grid + (r even ? w : grid - 1 - w), which balances the causal work across rounds."""
    e = gen.emit
    T0, T1, T2, T3 = (sr(S_T0), sr(S_T1), sr(S_T2), sr(S_T3))
    e(I(".Lblock:"))
    # every wave has finished the previous block's LDS reads before its stages are refilled
    e(I("s_barrier"))
    grid = arg("grid")
    e([I(f"s_mul_i32 {T0}, {sr(S_ROUND)}, {grid}"),
       I(f"s_sub_u32 {T1}, {grid}, 1"),
       I(f"s_sub_u32 {T1}, {T1}, s2"),
       I(f"s_bitcmp1_b32 {sr(S_ROUND)}, 0"),              # (after the subtractions: SCC)
       I(f"s_cselect_b32 {T1}, {T1}, s2"),
       I(f"s_add_u32 {T0}, {T0}, {T1}"),                      # o
       I(f"s_cmp_ge_u32 {T0}, {arg('nb')}"),
       I("s_cbranch_scc0 .Lhave_block"),
       I("s_endpgm"),
       I(".Lhave_block:")])
    e(fdiv(T1, T0, arg("fd_units_m"), arg("fd_units_s"), T3))   # rank = o / units
    e([I(f"s_mul_i32 {T2}, {T1}, {arg('units')}"),
       I(f"s_sub_u32 {sr(S_BH)}, {T0}, {T2}"),                 # bh = o % units
       I(f"s_sub_u32 {sr(S_QB)}, {arg('nqb')}, 1"),
       I(f"s_sub_u32 {sr(S_QB)}, {sr(S_QB)}, {T1}")])
    e(fdiv(sr(S_B), sr(S_BH), arg("fd_kvh_m"), arg("fd_kvh_s"), T3))
    e([I(f"s_mul_i32 {T1}, {sr(S_B)}, {arg('kv_heads')}"),
       I(f"s_sub_u32 {sr(S_KVH)}, {sr(S_BH)}, {T1}"),
       # a block beyond the batch (never produced by the host's arguments) exits before any access
       I(f"s_cmp_ge_u32 {sr(S_B)}, {arg('batch')}"),
       I("s_cbranch_scc0 .Lbatch_ok"),
       I("s_endpgm"),
       I(".Lbatch_ok:")])

    # ---- tile counts of the block: rows qb*256 .. +255
    gs = arg("gshift")
    e([I(f"s_lshl_b32 {T0}, {sr(S_QB)}, 8"),               # first row
       I(f"s_lshr_b32 {T1}, {T0}, {gs}"),                   # t_min
       I(f"s_add_u32 {T2}, {T0}, 255"),
       I(f"s_lshr_b32 {T2}, {T2}, {gs}"),
       I(f"s_sub_u32 {T3}, {arg('q_len')}, 1"),
       I(f"s_min_u32 {T2}, {T2}, {T3}"),                    # t_max
       I(f"s_add_u32 {T2}, {T2}, {arg('causal_off')}"),
       I(f"s_add_u32 {T2}, {T2}, 1"),                       # keys a causal block needs
       I(f"s_min_u32 {T2}, {T2}, {arg('kv_len')}"),
       I(f"s_cmp_eq_u32 {arg('causal')}, 0"),
       I(f"s_cselect_b32 {T2}, {arg('kv_len')}, {T2}"),
       I(f"s_add_u32 {T2}, {T2}, 63"),
       I(f"s_lshr_b32 {sr(S_N)}, {T2}, 6"),                 # n tiles
       I(f"s_lshr_b32 {T3}, {arg('kv_len')}, 6"),           # tiles without a tail
       I(f"s_add_u32 {T1}, {T1}, {arg('causal_off')}"),
       I(f"s_add_u32 {T1}, {T1}, 1"),
       I(f"s_lshr_b32 {T1}, {T1}, 6"),
       I(f"s_cmp_eq_u32 {arg('causal')}, 0"),
       I(f"s_cselect_b32 {T1}, {T3}, {T1}"),
       I(f"s_min_u32 {sr(S_NFULL)}, {T1}, {T3}"),
       I(f"s_sub_u32 {sr(S_NM1)}, {sr(S_N)}, 1"),
       # unmasked loop iterations: j < min(n - 1, nfull - 1)
       I(f"s_sub_u32 {T1}, {sr(S_NFULL)}, 1"),
       I(f"s_cmp_lt_i32 {T1}, 0"),
       I(f"s_cselect_b32 {T1}, 0, {T1}"),
       I(f"s_min_u32 {sr(S_JU)}, {T1}, {sr(S_NM1)}")])

    # ---- per-lane rows: row = r0 + 32 rb + (lane & 31); t = row >> gshift; head = row & (G-1)
    e([I(f"s_lshl_b32 {T0}, {sr(S_QB)}, 8"),
       I(f"s_lshl_b32 {T1}, {sr(S_WAVE)}, 6"),
       I(f"s_add_u32 {T0}, {T0}, {T1}"),                    # wave's first row
       I(f"s_lshl_b32 {T2}, {arg('q_len')}, {gs}"),         # rows_total
       I(f"s_lshl_b32 {T3}, 1, {gs}"),
       I(f"s_sub_u32 {T3}, {T3}, 1"),                       # group - 1
       I(f"v_and_b32 {vr(V_ROW + 3)}, 31, {vr(V_LANE)}")])
    for rb in range(2):
        row, t, hd, ok = V_ROW, V_ROW + 1, V_ROW + 2, None
        e([I(f"v_add_u32 {vr(row)}, {T0}, {vr(V_ROW + 3)}"),
           I(f"v_add_u32 {vr(row)}, {32 * rb}, {vr(row)}"),
           I(f"v_cmp_gt_u32 vcc, {T2}, {vr(row)}", reads=[T2, f"v{row}"], writes=["vcc"]),
           I(f"v_lshrrev_b32 {vr(t)}, {gs}, {vr(row)}"),
           I(f"v_and_b32 {vr(hd)}, {T3}, {vr(row)}"),
           I(f"s_sub_u32 {T1}, {arg('q_len')}, 1"),
           I(f"v_mov_b32 {vr(V_TMP)}, {T1}"),
           I(f"v_cndmask_b32 {vr(t)}, {vr(V_TMP)}, {vr(t)}, vcc",
             reads=[f"v{V_TMP}", f"v{t}", "vcc"], writes=[f"v{t}"]),
           I(f"v_cndmask_b32 {vr(hd)}, 0, {vr(hd)}, vcc", reads=[f"v{hd}", "vcc"],
             writes=[f"v{hd}"]),
           # O and LSE offsets (INVALID for rows past the sequence); LSE only from lanes < 32
           I(f"v_mul_lo_u32 {vr(V_OOFF + rb)}, {vr(hd)}, {arg('o_sh')}"),
           I(f"v_mul_lo_u32 {vr(V_TMP + 1)}, {vr(t)}, {arg('o_ss')}"),
           I(f"v_add_u32 {vr(V_OOFF + rb)}, {vr(V_OOFF + rb)}, {vr(V_TMP + 1)}"),
           I(f"v_mul_lo_u32 {vr(V_LOFF + rb)}, {vr(hd)}, {arg('lse_sh')}"),
           I(f"v_lshl_add_u32 {vr(V_LOFF + rb)}, {vr(t)}, 2, {vr(V_LOFF + rb)}"),
           I(f"v_mov_b32 {vr(V_TMP + 2)}, 0x{INVALID_OFF:x}"),
           I(f"v_cndmask_b32 {vr(V_OOFF + rb)}, {vr(V_TMP + 2)}, {vr(V_OOFF + rb)}, vcc",
             reads=[f"v{V_TMP + 2}", f"v{V_OOFF + rb}", "vcc"], writes=[f"v{V_OOFF + rb}"]),
           I(f"v_cndmask_b32 {vr(V_LOFF + rb)}, {vr(V_TMP + 2)}, {vr(V_LOFF + rb)}, vcc",
             reads=[f"v{V_TMP + 2}", f"v{V_LOFF + rb}", "vcc"], writes=[f"v{V_LOFF + rb}"]),
           # Q offset: head * q_sh + t * q_ss + 16 g
           I(f"v_mul_lo_u32 {vr(V_QOFF + rb)}, {vr(hd)}, {arg('q_sh')}"),
           I(f"v_mul_lo_u32 {vr(V_TMP + 1)}, {vr(t)}, {arg('q_ss')}"),
           I(f"v_add_u32 {vr(V_QOFF + rb)}, {vr(V_QOFF + rb)}, {vr(V_TMP + 1)}"),
           # (cos, sin) row of position q_rope_off + t: 512 bytes per position (64 pairs)
           I(f"v_add_u32 {vr(V_CSOFF + rb)}, {arg('q_rope_off')}, {vr(t)}"),
           I(f"v_lshlrev_b32 {vr(V_CSOFF + rb)}, 9, {vr(V_CSOFF + rb)}"),
           # limit base: (causal ? min(kv_len - 1, causal_off + t) : kv_len - 1) - 8 g
           I(f"s_sub_u32 {T1}, {arg('kv_len')}, 1"),
           I(f"v_add_u32 {vr(V_LIMB + rb)}, {arg('causal_off')}, {vr(t)}"),
           I(f"v_min_i32 {vr(V_LIMB + rb)}, {T1}, {vr(V_LIMB + rb)}"),
           I(f"v_mov_b32 {vr(V_TMP + 1)}, {T1}"),
           I(f"s_cmp_eq_u32 {arg('causal')}, 0"),
           I(f"s_cselect_b64 vcc, -1, 0", writes=["vcc"]),
           I("s_nop 1"),
           I(f"v_cndmask_b32 {vr(V_LIMB + rb)}, {vr(V_LIMB + rb)}, {vr(V_TMP + 1)}, vcc",
             reads=[f"v{V_LIMB + rb}", f"v{V_TMP + 1}", "vcc"], writes=[f"v{V_LIMB + rb}"])])
    # g-dependent parts: +16 g bytes (Q, O), 8 g keys off the limit, LSE stores only from g == 0
    e([I(f"v_lshrrev_b32 {vr(V_ROW)}, 5, {vr(V_LANE)}"),          # g
       I(f"v_lshlrev_b32 {vr(V_ROW + 1)}, 4, {vr(V_ROW)}"),       # 16 g
       I(f"v_lshlrev_b32 {vr(V_ROW + 2)}, 3, {vr(V_ROW)}"),       # 8 g
       I(f"v_cmp_eq_u32 vcc, 0, {vr(V_ROW)}", reads=[f"v{V_ROW}"], writes=["vcc"]),
       I(f"v_mov_b32 {vr(V_TMP + 2)}, 0x{INVALID_OFF:x}")])
    for rb in range(2):
        e([I(f"v_add_u32 {vr(V_QOFF + rb)}, {vr(V_QOFF + rb)}, {vr(V_ROW + 1)}"),
           I(f"v_add_u32 {vr(V_CSOFF + rb)}, {vr(V_CSOFF + rb)}, {vr(V_ROW + 1)}"),
           I(f"v_add_u32 {vr(V_CSOFF + rb)}, {vr(V_CSOFF + rb)}, {vr(V_ROW + 1)}"),
           I(f"v_sub_u32 {vr(V_LIMB + rb)}, {vr(V_LIMB + rb)}, {vr(V_ROW + 2)}"),
           I(f"v_cndmask_b32 {vr(V_LOFF + rb)}, {vr(V_TMP + 2)}, {vr(V_LOFF + rb)}, vcc",
             reads=[f"v{V_TMP + 2}", f"v{V_LOFF + rb}", "vcc"], writes=[f"v{V_LOFF + rb}"]),
           # O: the lane writes dims mb*32 + 8 q4 + 4 g: + 8 g bytes, skip if row invalid
           I(f"v_cmp_ne_u32 {sr(S_NEED0, 2)}, {vr(V_TMP + 2)}, {vr(V_OOFF + rb)}",
             reads=[f"v{V_OOFF + rb}", f"v{V_TMP + 2}"], writes=[f"s{S_NEED0}", f"s{S_NEED0 + 1}"]),
           I(f"v_add_u32 {vr(V_TMP + 3)}, {vr(V_OOFF + rb)}, {vr(V_ROW + 2)}"),
           I(f"v_cndmask_b32_e64 {vr(V_OOFF + rb)}, {vr(V_OOFF + rb)}, {vr(V_TMP + 3)}, "
             f"{sr(S_NEED0, 2)}", reads=[f"v{V_OOFF + rb}", f"v{V_TMP + 3}", f"s{S_NEED0}",
                                         f"s{S_NEED0 + 1}"], writes=[f"v{V_OOFF + rb}"])])
    # ---- base addresses: K/V of (b, kvh); Q/O/LSE of (b, first head of the group)
    def base64(dst, ptr, sb, sh_lo, sh_hi, headmul):
        # dst = ptr + b * sb + headmul * sh   (64-bit)
        return [I(f"s_mul_i32 {T0}, {sr(S_B)}, {arg(sb)}"),
                I(f"s_mul_hi_u32 {T1}, {sr(S_B)}, {arg(sb)}"),
                I(f"s_mul_i32 {T2}, {sr(S_B)}, {arg(sb, True)}"),
                I(f"s_add_u32 {T1}, {T1}, {T2}"),
                I(f"s_add_u32 {sr(dst)}, {arg(ptr)}, {T0}"),
                I(f"s_addc_u32 {sr(dst + 1)}, {arg(ptr, True)}, {T1}"),
                I(f"s_mul_i32 {T0}, {headmul}, {sh_lo}"),
                I(f"s_mul_hi_u32 {T1}, {headmul}, {sh_lo}")] + \
               ([I(f"s_mul_i32 {T2}, {headmul}, {sh_hi}"), I(f"s_add_u32 {T1}, {T1}, {T2}")]
                if sh_hi else []) + \
               [I(f"s_add_u32 {sr(dst)}, {sr(dst)}, {T0}"),
                I(f"s_addc_u32 {sr(dst + 1)}, {sr(dst + 1)}, {T1}")]
    if PAGED:
        # K/V of this kv head in the page pool (no batch term: pages come from the tables)
        for dst, ptr in ((S_KBASE, "k"), (S_VBASE, "v")):
            e([I(f"s_mul_i32 {T0}, {sr(S_KVH)}, {arg('k_sh')}"),
               I(f"s_mul_hi_u32 {T1}, {sr(S_KVH)}, {arg('k_sh')}"),
               I(f"s_mul_i32 {T2}, {sr(S_KVH)}, {arg('k_sh', True)}"),
               I(f"s_add_u32 {T1}, {T1}, {T2}"),
               I(f"s_add_u32 {sr(dst)}, {arg(ptr)}, {T0}"),
               I(f"s_addc_u32 {sr(dst + 1)}, {arg(ptr, True)}, {T1}")])
    else:
        e(base64(S_KBASE, "k", "k_sb", arg("k_sh"), arg("k_sh", True), sr(S_KVH)))
        e(base64(S_VBASE, "v", "k_sb", arg("k_sh"), arg("k_sh", True), sr(S_KVH)))
        # nrec_all = (kv_len - 1) * row_bytes + 256
        e([I(f"s_sub_u32 {T0}, {arg('kv_len')}, 1"),
           I(f"s_mul_i32 {sr(S_NREC)}, {T0}, {arg('k_ss')}"),
           I(f"s_add_u32 {sr(S_NREC)}, {sr(S_NREC)}, 256")])
    # transfer offsets: instruction i covers rows 16 wave + 4 i + (lane >> 4) of the tile (LDS
    # KiB 4 wave + i; paged: in-page rows 4 i + (lane >> 4) of page `wave`, whose resource the
    # transfer code bases at the page); slot chunk lane & 15 holds global chunk
    # (lane & 15) ^ (4 (lane >> 4) + i), less the instruction offset 1024 i
    e([I(f"v_lshrrev_b32 {vr(V_ROW)}, 4, {vr(V_LANE)}"),           # lane >> 4
       I(f"v_and_b32 {vr(V_ROW + 1)}, 15, {vr(V_LANE)}"),
       I(f"v_lshlrev_b32 {vr(V_ROW + 2)}, 2, {vr(V_ROW)}")])        # 4 (lane >> 4)
    # row of instruction 0 (paged: in-page, no wave term)
    e([I(f"v_mov_b32 {vr(V_ROW + 3)}, {vr(V_ROW)}")] if PAGED else
      [I(f"s_lshl_b32 {T0}, {sr(S_WAVE)}, 4"),
       I(f"v_add_u32 {vr(V_ROW + 3)}, {T0}, {vr(V_ROW)}")])
    for i in range(4):
        e([I(f"v_add_u32 {vr(V_TMP)}, {4 * i}, {vr(V_ROW + 3)}"),
           I(f"v_mul_lo_u32 {vr(VTOFF + i)}, {vr(V_TMP)}, {arg('k_ss')}"),
           I(f"v_add_u32 {vr(V_TMP + 1)}, {i}, {vr(V_ROW + 2)}"),
           I(f"v_xor_b32 {vr(V_TMP + 1)}, {vr(V_TMP + 1)}, {vr(V_ROW + 1)}"),  # global chunk
           I(f"v_lshlrev_b32 {vr(V_TMP + 1)}, 4, {vr(V_TMP + 1)}"),
           I(f"v_add_u32 {vr(VTOFF + i)}, {vr(VTOFF + i)}, {vr(V_TMP + 1)}"),
           I(f"v_add_u32 {vr(VTOFF + i)}, 0x{(-1024 * i) & 0xffffffff:x}, {vr(VTOFF + i)}")])
    # K read addresses (stage 0): row p = perm(lane & 31) (bits 2, 3 swapped),
    # chunk (2 ks + g) ^ swz(p); V^T read addresses (stage 0, V region at +16 KiB)
    e([I(f"v_and_b32 {vr(V_ROW)}, 31, {vr(V_LANE)}"),
       I(f"v_and_b32 {vr(V_ROW + 1)}, 0x13, {vr(V_ROW)}"),
       I(f"v_bfe_u32 {vr(V_ROW + 2)}, {vr(V_ROW)}, 2, 1"),
       I(f"v_lshl_or_b32 {vr(V_ROW + 1)}, {vr(V_ROW + 2)}, 3, {vr(V_ROW + 1)}"),
       I(f"v_bfe_u32 {vr(V_ROW + 2)}, {vr(V_ROW)}, 3, 1"),
       I(f"v_lshl_or_b32 {vr(V_ROW + 1)}, {vr(V_ROW + 2)}, 2, {vr(V_ROW + 1)}"),  # p
       # swz(p) = 4 (p & 3) + ((p >> 2) & 3)
       I(f"v_and_b32 {vr(V_ROW + 2)}, 3, {vr(V_ROW + 1)}"),
       I(f"v_bfe_u32 {vr(V_ROW + 3)}, {vr(V_ROW + 1)}, 2, 2"),
       I(f"v_lshl_or_b32 {vr(V_ROW + 2)}, {vr(V_ROW + 2)}, 2, {vr(V_ROW + 3)}"),
       I(f"v_lshrrev_b32 {vr(V_ROW + 3)}, 5, {vr(V_LANE)}"),      # g
       I(f"v_xor_b32 {vr(V_ROW + 2)}, {vr(V_ROW + 2)}, {vr(V_ROW + 3)}"),  # g ^ swz(p)
       I(f"v_lshlrev_b32 {vr(V_ROW + 1)}, 8, {vr(V_ROW + 1)}")])  # p * 256
    for ks in range(8):
        e([I(f"v_xor_b32 {vr(V_TMP)}, {2 * ks}, {vr(V_ROW + 2)}"),
           I(f"v_lshl_add_u32 {vr(VKA + ks)}, {vr(V_TMP)}, 4, {vr(V_ROW + 1)}")])
    # V^T: row = 8 g + ((lane & 15) >> 2) (+4 for hi); chunk 4 mb + 2 ((lane >> 4) & 1) +
    # ((lane & 3) >> 1); byte 8 (lane & 1)
    e([I(f"v_lshrrev_b32 {vr(V_ROW)}, 5, {vr(V_LANE)}"),
       I(f"v_bfe_u32 {vr(V_ROW + 1)}, {vr(V_LANE)}, 2, 2"),
       I(f"v_lshl_add_u32 {vr(V_ROW)}, {vr(V_ROW)}, 3, {vr(V_ROW + 1)}"),   # row lo
       I(f"v_bfe_u32 {vr(V_ROW + 1)}, {vr(V_LANE)}, 4, 1"),
       I(f"v_bfe_u32 {vr(V_ROW + 2)}, {vr(V_LANE)}, 1, 1"),
       I(f"v_lshl_or_b32 {vr(V_ROW + 1)}, {vr(V_ROW + 1)}, 1, {vr(V_ROW + 2)}"),  # chunk low
       I(f"v_and_b32 {vr(V_ROW + 2)}, 1, {vr(V_LANE)}"),
       I(f"v_lshlrev_b32 {vr(V_ROW + 2)}, 3, {vr(V_ROW + 2)}")])              # byte in chunk
    for mb in range(4):
        for hi in range(2):
            # row r = rowlo + 4 hi; swz(r); addr = 16 KiB + r * 256 + 16 ((4 mb + cl) ^ swz) + byte
            e([I(f"v_add_u32 {vr(V_TMP)}, {4 * hi}, {vr(V_ROW)}"),
               I(f"v_and_b32 {vr(V_TMP + 1)}, 3, {vr(V_TMP)}"),
               I(f"v_bfe_u32 {vr(V_TMP + 2)}, {vr(V_TMP)}, 2, 2"),
               I(f"v_lshl_or_b32 {vr(V_TMP + 1)}, {vr(V_TMP + 1)}, 2, {vr(V_TMP + 2)}"),
               I(f"v_add_u32 {vr(V_TMP + 2)}, {4 * mb}, {vr(V_ROW + 1)}"),
               I(f"v_xor_b32 {vr(V_TMP + 1)}, {vr(V_TMP + 1)}, {vr(V_TMP + 2)}"),
               I(f"v_lshlrev_b32 {vr(V_TMP + 1)}, 4, {vr(V_TMP + 1)}"),
               I(f"v_lshl_add_u32 {vr(V_TMP)}, {vr(V_TMP)}, 8, {vr(V_TMP + 1)}"),
               I(f"v_add_u32 {vr(V_TMP)}, {vr(V_TMP)}, {vr(V_ROW + 2)}"),
               I(f"v_add_u32 {vr(VVA + mb * 2 + hi)}, 0x{V_REGION():x}, {vr(V_TMP)}")])
    # ---- transfers of tiles 0 .. 2 into stages 0 .. 2 (paged: after the Q loads, once the
    # page ids of tiles 0 .. 2 have landed)
    e(I(f"s_mov_b32 {sr(S_TSLOT)}, 0"))
    e(I(f"s_mov_b32 {sr(S_TT)}, 0"))
    if PAGED:
        e(bt_resource())
        e(pt_load(sr(S_TT)))
    # ---- Q rows into AGPRs, rotated when rope_q
    # Q resource base = q + b * q_sb + (kvh << gshift) * q_sh
    e([I(f"s_lshl_b32 {sr(S_T3)}, {sr(S_KVH)}, {gs}")])
    e([I(f"s_mul_i32 {T0}, {sr(S_B)}, {arg('q_sb')}"),
       I(f"s_mul_hi_u32 {T1}, {sr(S_B)}, {arg('q_sb')}"),
       I(f"s_mul_i32 {T2}, {sr(S_B)}, {arg('q_sb', True)}"),
       I(f"s_add_u32 {T1}, {T1}, {T2}"),
       I(f"s_add_u32 {sr(S_RQ)}, {arg('q')}, {T0}"),
       I(f"s_addc_u32 {sr(S_RQ + 1)}, {arg('q', True)}, {T1}"),
       I(f"s_mul_i32 {T0}, {T3}, {arg('q_sh')}"),
       I(f"s_mul_hi_u32 {T1}, {T3}, {arg('q_sh')}"),
       I(f"s_add_u32 {sr(S_RQ)}, {sr(S_RQ)}, {T0}"),
       I(f"s_addc_u32 {sr(S_RQ + 1)}, {sr(S_RQ + 1)}, {T1}"),
       I(f"s_and_b32 {sr(S_RQ + 1)}, {sr(S_RQ + 1)}, 0xffff"),
       I(f"s_mov_b32 {sr(S_RQ + 2)}, {sr(S_QNREC)}"),
       I(f"s_mov_b32 {sr(S_RQ + 3)}, 0x20000")])
    # Q^T operands: Q rotated (rope_q) and scaled by c2, rounded once to bf16, into AGPRs.
    # Loads: both blocks' Q rows first, then the (cos, sin) rows in four batches of four 16-dim
    # chunks alternating between two register areas, each batch's rotation overlapping the next
    # batch's loads.
    RT = S_T0
    qt = [SB[0], SB[1]]          # 32 registers of Q per block (8 chunks x 4)
    cs_area = [PB[0], NB]        # 32 registers each: 4 chunks x 8 (cos, sin)
    for rb in range(2):
        for ks in range(8):
            e(I(f"buffer_load_dwordx4 {vr(qt[rb] + 4 * ks, 4)}, {vr(V_QOFF + rb)}, {sr(S_RQ, 4)}, 0 "
                f"offen offset:{32 * ks}"))
    def tile_transfers(pending: int) -> int:
        """The transfers of tiles 0 .. 2 into stages 0 .. 2, issued after the Q loads and the
        first (cos, sin) loads so that those reach the rotation first. Paged: once the page ids
        of tiles 0 .. 2 (issued before the Q loads, `pending` loads ago) have landed, then the
        page ids of tiles 3 and 4 for the first pair of the loop (S_RQ: the block-table row
        again; the Q loads have read their resource). Returns the loads issued."""
        if PAGED:
            assert PAIR
            e(I(f"s_waitcnt vmcnt({pending})"))
            for t in range(3):
                e(transfer_paged(sr(S_TT), 4 * t))
                e([I(f"s_add_u32 {sr(S_TT)}, {sr(S_TT)}, 1"),
                   I(f"s_add_u32 {sr(S_TSLOT)}, {sr(S_TSLOT)}, 1")])
            e(bt_resource())
            e(pt_load(sr(S_TT)))
            return 3 * 8 + 1
        for _ in range(3 if PAIR else 2):
            e(transfer_setup(sr(S_TT)))
            e(kv_transfers())
            e([I(f"s_add_u32 {sr(S_TT)}, {sr(S_TT)}, 1"),
               I(f"s_add_u32 {sr(S_TSLOT)}, {sr(S_TSLOT)}, 1")])
        return (3 if PAIR else 2) * (12 if PREC else 8)
    c2 = arg("c2")

    def residual(w, t1, od, lo_a):
        """Precise kernel: a[lo_a] = bf16 residuals of the f32 pair (t1, od) rounded into w."""
        if not PREC:
            return []
        ev = V_TMP + 3
        return [I(f"v_lshlrev_b32 {vr(ev)}, 16, {vr(w)}"),
                I(f"v_sub_f32 {vr(t1)}, {vr(t1)}, {vr(ev)}"),
                I(f"v_and_b32 {vr(ev)}, 0xffff0000, {vr(w)}"),
                I(f"v_sub_f32 {vr(od)}, {vr(od)}, {vr(ev)}"),
                I(f"v_cvt_pk_bf16_f32 {vr(ev)}, {vr(t1)}, {vr(od)}"),
                I(f"v_accvgpr_write_b32 {ar(lo_a)}, {vr(ev)}")]

    def rotate_chunk(w0, cs0, lo_a0):
        out = []
        for j in range(4):
            w = w0 + j
            c, sn = cs0 + 2 * j, cs0 + 2 * j + 1
            ev, od, t1 = V_TMP, V_TMP + 1, V_TMP + 2
            out += unpack(vr(ev), vr(od), vr(w))
            out += [I(f"v_mul_f32 {vr(t1)}, {vr(od)}, {vr(sn)}"),
                    I(f"v_fma_f32 {vr(t1)}, {vr(ev)}, {vr(c)}, -{vr(t1)}"),
                    I(f"v_mul_f32 {vr(od)}, {vr(od)}, {vr(c)}"),
                    I(f"v_fma_f32 {vr(od)}, {vr(ev)}, {vr(sn)}, {vr(od)}"),
                    I(f"v_mul_f32 {vr(t1)}, {c2}, {vr(t1)}"),
                    I(f"v_mul_f32 {vr(od)}, {c2}, {vr(od)}"),
                    I(f"{CVT()} {vr(w)}, {vr(t1)}, {vr(od)}")]
            out += residual(w, t1, od, lo_a0 + j)
        return out

    e(I(f"s_cmp_eq_u32 {arg('rope_q')}, 0"))
    e(I("s_cbranch_scc1 .Lq_norope"))
    rt_set = [I(f"s_mov_b32 {sr(RT)}, {arg('rope')}"),
              I(f"s_and_b32 {sr(RT + 1)}, {arg('rope', True)}, 0xffff"),
              I(f"s_mov_b32 {sr(RT + 2)}, {arg('rope_bytes')}"),
              I(f"s_mov_b32 {sr(RT + 3)}, 0x20000")]
    e(rt_set)

    def cs_batch(bi):
        rb, k0 = bi // 2, 4 * (bi % 2)
        area = cs_area[bi % 2]
        return [I(f"buffer_load_dwordx4 {vr(area + 8 * k + 4 * h, 4)}, {vr(V_CSOFF + rb)}, "
                  f"{sr(RT, 4)}, 0 offen offset:{64 * (k0 + k) + 16 * h}")
                for k in range(4) for h in range(2)]

    e(cs_batch(0))
    e(cs_batch(1))
    # (paged: the page-id load of tiles 0 .. 2 precedes the 16 Q and 16 (cos, sin) loads)
    x = tile_transfers(32)
    e(rt_set)  # (the transfer code used the temps RT overlays)
    # batches 0 and 1 wait for everything but the loads issued after them (cs1 and the
    # transfers, then the transfers and cs2); batch 2 also for the transfers
    for bi in range(4):
        rb, k0 = bi // 2, 4 * (bi % 2)
        e(I(f"s_waitcnt vmcnt({(8 + x) if bi < 2 else (8 if bi == 2 else 0)})"))
        for k in range(4):
            e(rotate_chunk(qt[rb] + 4 * (k0 + k), cs_area[bi % 2] + 8 * k,
                           A_QLO + rb * 32 + 4 * (k0 + k)))
        if bi + 2 < 4:
            e(cs_batch(bi + 2))
    e(I("s_branch .Lq_done"))
    e(I(".Lq_norope:"))
    tile_transfers(16)
    e(I("s_waitcnt vmcnt(0)"))
    for rb in range(2):
        for w in range(32):
            r = qt[rb] + w
            ev, od = V_TMP, V_TMP + 1
            e(unpack(vr(ev), vr(od), vr(r)))
            e([I(f"v_mul_f32 {vr(ev)}, {c2}, {vr(ev)}"),
               I(f"v_mul_f32 {vr(od)}, {c2}, {vr(od)}"),
               I(f"{CVT()} {vr(r)}, {vr(ev)}, {vr(od)}")])
            e(residual(r, ev, od, A_QLO + rb * 32 + w))
    e(I(".Lq_done:"))
    e(I("s_waitcnt vmcnt(0)"))
    for rb in range(2):
        for w in range(32):
            e(I(f"v_accvgpr_write_b32 {ar(A_Q + rb * 32 + w)}, {vr(qt[rb] + w)}"))
    # ---- O = 0 (eight MFMAs of zero operands write the 128 accumulators: 8 instructions
    # instead of 128 AGPR writes), running statistics
    e([I(f"v_mov_b32 {vr(NB + i)}, 0") for i in range(4)])
    for blk in range(8):
        e(I(f"{MF()} {ar(A_O + 16 * blk, 16)}, {vr(NB, 4)}, {vr(NB, 4)}, 0"))
    for rb in range(2):
        e([I(f"v_mov_b32 {vr(V_M + rb)}, 0xff800000"),
           I(f"v_mov_b32 {vr(V_L + rb)}, 0")])
    e(I(f"s_mov_b32 {sr(S_KSLOT)}, 0"))
    e(I(f"s_mov_b32 {sr(S_VSLOT)}, 0"))
    e(I("s_waitcnt vmcnt(0)"))
    # tiles 2 .. NSTAGE - 2 (their waits come at the ends of the first iterations)
    for _ in range(0 if PAIR else NSTAGE - 3):
        e(transfer_setup(sr(S_TT)))
        e(kv_transfers())
        e([I(f"s_add_u32 {sr(S_TT)}, {sr(S_TT)}, 1"),
           I(f"s_add_u32 {sr(S_TSLOT)}, {sr(S_TSLOT)}, 1")])
    e(I("s_barrier"))


def epilogue_store(gen: Gen):
    e = gen.emit
    # l_tot = l + l(partner); LSE = m * scale + ln l_tot; inv = 1 / l_tot
    for rb in range(2):
        a, b = V_MX, V_MX + 1
        e([I(f"v_mov_b32 {vr(a)}, {vr(V_L + rb)}"),
           I(f"v_mov_b32 {vr(b)}, {vr(V_L + rb)}"),
           I(f"v_permlane32_swap_b32 {vr(a)}, {vr(b)}"),
           I(f"v_cndmask_b32_e64 {vr(b)}, {vr(b)}, {vr(a)}, {sr(S_HIMASK, 2)}",
             reads=[f"v{a}", f"v{b}", f"s{S_HIMASK}", f"s{S_HIMASK + 1}"], writes=[f"v{b}"]),
           I(f"v_add_f32 {vr(V_L + rb)}, {vr(V_L + rb)}, {vr(b)}"),
           I(f"v_rcp_f32 {vr(V_ALPHA + rb)}, {vr(V_L + rb)}"),
           I(f"v_log_f32 {vr(V_U + rb)}, {vr(V_L + rb)}"),
           I(f"v_add_f32 {vr(V_U + rb)}, {vr(V_U + rb)}, {vr(V_M + rb)}"),
           I(f"v_mul_f32 {vr(V_U + rb)}, 0x3f317218, {vr(V_U + rb)}")])
    # O/LSE resources
    T0, T1, T2, T3 = (sr(S_T0), sr(S_T1), sr(S_T2), sr(S_T3))
    gs = arg("gshift")

    def res(dst, ptr, sb, sh, nrec):
        return [I(f"s_lshl_b32 {T3}, {sr(S_KVH)}, {gs}"),
                I(f"s_mul_i32 {T0}, {sr(S_B)}, {arg(sb)}"),
                I(f"s_mul_hi_u32 {T1}, {sr(S_B)}, {arg(sb)}"),
                I(f"s_mul_i32 {T2}, {sr(S_B)}, {arg(sb, True)}"),
                I(f"s_add_u32 {T1}, {T1}, {T2}"),
                I(f"s_add_u32 {sr(dst)}, {arg(ptr)}, {T0}"),
                I(f"s_addc_u32 {sr(dst + 1)}, {arg(ptr, True)}, {T1}"),
                I(f"s_mul_i32 {T0}, {T3}, {arg(sh)}"),
                I(f"s_mul_hi_u32 {T1}, {T3}, {arg(sh)}"),
                I(f"s_add_u32 {sr(dst)}, {sr(dst)}, {T0}"),
                I(f"s_addc_u32 {sr(dst + 1)}, {sr(dst + 1)}, {T1}"),
                I(f"s_and_b32 {sr(dst + 1)}, {sr(dst + 1)}, 0xffff"),
                I(f"s_mov_b32 {sr(dst + 2)}, {sr(nrec)}"),
                I(f"s_mov_b32 {sr(dst + 3)}, 0x20000")]
    e(res(S_RQ, "o", "o_sb", "o_sh", S_ONREC))
    e(res(S_RK, "lse", "lse_sb", "lse_sh", S_LNREC))
    for rb in range(2):
        e(I(f"buffer_store_dword {vr(V_U + rb)}, {vr(V_LOFF + rb)}, {sr(S_RK, 4)}, 0 offen"))
    # O goes out through LDS so that every store instruction writes whole rows: written from the
    # accumulators a lane holds 4 dims of one row (32 rows per instruction, partial lines), read
    # back 16 lanes cover one 256-byte row. The staging area (the first 4 * O_WAVEB bytes) overlays
    # the K/V stages: the barrier retires every wave's reads of this block's tiles, no transfer is
    # in flight (the last one was waited for before the loop's last barrier), and the next block
    # refills the stages only after its opening barrier, when these reads have completed.
    e(I("s_barrier"))
    W, R, P, C = V_EPI, V_EPI + 1, V_EPI + 2, V_EPI + 3
    DATA = SB[0]                 # 64 registers: bf16 pairs to stage, then the rows read back
    n = 0
    for rb in range(2):
        for mb in range(4):
            for q4 in range(4):
                regs = [A_O + (rb * 4 + mb) * 16 + 4 * q4 + i for i in range(4)]
                t = V_TMP
                d = DATA + 2 * n
                e([I(f"v_accvgpr_read_b32 {vr(t + i)}, {ar(a)}") for i, a in enumerate(regs)])
                e([I(f"v_mul_f32 {vr(t + i)}, {vr(t + i)}, {vr(V_ALPHA + rb)}") for i in range(4)])
                e([I(f"{CVT()} {vr(d)}, {vr(t)}, {vr(t + 1)}"),
                   I(f"{CVT()} {vr(d + 1)}, {vr(t + 2)}, {vr(t + 3)}")])
                e(I(f"ds_write_b64 {vr(W)}, {vr(d, 2)} "
                    f"offset:{rb * 32 * O_ROWB + mb * 64 + 16 * q4}"))
                n += 1
    e(I("s_waitcnt lgkmcnt(0)"))
    # rows 4 i .. 4 i + 3 of the wave per store: the byte offset of row 4 i + (lane >> 4) is
    # V_OOFF of the lane that held it (rows 0..31: lane r of rb 0, rows 32..63: lane r - 32 of
    # rb 1; lanes 0..31 hold it without the 8 g term, INVALID for rows past the sequence)
    PERM, SOFF = PB[0], PB[1]
    for batch in range(4):
        for k in range(4):
            i = 4 * batch + k
            rb = i // 8
            e(I(f"ds_bpermute_b32 {vr(PERM + i)}, {vr(P)}, {vr(V_OOFF + rb)} offset:{16 * (i % 8)}"))
            e(I(f"ds_read_b128 {vr(DATA + 4 * i, 4)}, {vr(R)} offset:{i * 4 * O_ROWB}"))
        e(I("s_waitcnt lgkmcnt(0)"))
        for k in range(4):
            i = 4 * batch + k
            e(I(f"v_add_u32 {vr(SOFF + i)}, {vr(PERM + i)}, {vr(C)}"))
        for k in range(4):
            i = 4 * batch + k
            e(I(f"buffer_store_dwordx4 {vr(DATA + 4 * i, 4)}, {vr(SOFF + i)}, {sr(S_RQ, 4)}, 0 "
                "offen nt"))
    # next block of the persistent loop
    e([I(f"s_add_u32 {sr(S_ROUND)}, {sr(S_ROUND)}, 1"), I("s_branch .Lblock")])


# --------------------------------------------------------------------------- assembly of phases
def build() -> Gen:
    gen = Gen()
    gen.exact = []  # out-of-line exact paths: (tag, x, hh, s_x, branch block, continuation block)
    b_setup = gen.new_block("setup")
    setup(gen)
    b_block = gen.new_block("setup_block", [b_setup])
    setup_block(gen)
    # ---- prologue: S(0) alone (onto 0); its mask (only when tile 0 is not visible to every
    # row of the block) and row maxima set m and the bias blocks; then S(1) onto the bias with
    # the softmax of half-tile 0 spread over its MFMAs (no overflow: S' <= 0)
    gen.new_block("prologue", [b_block])
    gen.ds_outstanding = []
    phase(gen, pv_x=None, pv_hh=0, s_x=0, s_hh=0, sm_x=None, sm_masked=False, zero_bias=True)
    gen.ds_wait_all()
    gen.emit([I(f"s_mov_b32 {sr(S_KEY0)}, 0"),
              I(f"s_cmp_lg_u32 {sr(S_NFULL)}, 0"),
              I("s_cbranch_scc1 .Lpro_max")])
    br = gen.cur
    gen.new_block("pro_mask", [br])
    gen.emit(mask_program(0))
    mk = gen.cur
    gen.new_block("pro_max", [br, mk])
    gen.emit(I(".Lpro_max:"))
    first_max(gen, 0)
    phase(gen, pv_x=None, pv_hh=0, s_x=1, s_hh=1, sm_x=0, sm_masked=False, prefetch_v_hh=0,
          after_last_k=advance_slot(S_KSLOT, VKA, 8))
    gen.emit([I(f"v_mov_b32 {vr(V_L + rb)}, {vr(V_LT + rb)}") for rb in range(2)])
    pro_end = gen.cur
    if PAIR:
        epi_preds = pair_loops(gen, pro_end)
    else:
        epi_preds = single_loops(gen, pro_end)
    # ---- epilogue phases: P.V(2n-2) + softmax(2n-1) (masked), then P.V(2n-1)
    gen.new_block("epi", epi_preds)
    gen.emit(I(".Lepi:"))
    pre_ids = list(range(gen.ds_next, gen.ds_next + 2 * RV))
    gen.ds_next += 2 * RV
    gen.ds_outstanding = list(pre_ids)
    ring_in = {"ready": {o: pre_ids[2 * o:2 * o + 2] for o in range(RV)}}
    key_e = [I(f"s_lshl_b32 {sr(S_KEY0)}, {sr(S_NM1)}, 6"),
             I(f"s_add_u32 {sr(S_KEY0)}, {sr(S_KEY0)}, 32")]
    ring = phase(gen, pv_x=0, pv_hh=0, s_x=None, s_hh=0, sm_x=1, sm_masked=True,
                 pre=key_e, vring_state=ring_in, prefetch_v_hh=1)
    finish_phase(gen, "epi_a", 1, 1, None)
    ring = phase(gen, pv_x=1, pv_hh=1, s_x=None, s_hh=0, sm_x=None, sm_masked=False,
                 vring_state=ring)
    gen.ds_wait_all()
    epilogue_store(gen)
    b_block.preds.append(gen.cur)
    # ---- the out-of-line exact paths
    for tag, x, hh, s_x, br, cont in gen.exact:
        b = gen.new_block(f"exact_{tag}", [br])
        gen.emit(I(f".Lexact_{tag}:"))
        gen.ds_outstanding = [-1] * (2 * RV)
        exact_path(gen, x, hh, s_x)
        gen.emit(I(f"s_branch .Lcont_{tag}"))
        cont.preds.append(b)
    return gen


def single_loops(gen: Gen, pro_end: Block) -> list:
    """One barrier per iteration (NSTAGE >= 3 stages)."""
    gen.emit([I(f"s_mov_b32 {sr(S_J)}, 0"),
              I(f"s_cmp_ge_u32 {sr(S_J)}, {sr(S_JU)}"),
              I("s_cbranch_scc1 .Lmasked_check")])
    firsts, lasts = {}, {}
    for masked in (False, True):
        name = "loop_m" if masked else "loop_u"
        b = gen.new_block(name)
        firsts[masked] = b
        gen.emit(I(f".L{name}:"))
        pre_ids = list(range(gen.ds_next, gen.ds_next + 2 * RV))
        gen.ds_next += 2 * RV
        gen.ds_outstanding = list(pre_ids)
        ring_in = {"ready": {o: pre_ids[2 * o:2 * o + 2] for o in range(RV)}}
        # iteration j: transfer of tile j + NSTAGE - 1 into the stage of tile j - 1
        xfer = [I(f"s_add_u32 {sr(S_TT)}, {sr(S_J)}, {NSTAGE - 1}")] + \
            transfer_setup(sr(S_TT)) + kv_transfers() + \
            [I(f"s_add_u32 {sr(S_TSLOT)}, {sr(S_TSLOT)}, 1"),
             I(f"s_cmp_eq_u32 {sr(S_TSLOT)}, {NSTAGE}"),
             I(f"s_cselect_b32 {sr(S_TSLOT)}, 0, {sr(S_TSLOT)}")]
        key_a = [I(f"s_lshl_b32 {sr(S_KEY0)}, {sr(S_J)}, 6"),
                 I(f"s_add_u32 {sr(S_KEY0)}, {sr(S_KEY0)}, 32")]
        # phase 2j+1: P.V(2j) (PB0, V half 0), S(2j+2) (SB0, K half 0), softmax(2j+1) (SB1)
        ring = phase(gen, pv_x=0, pv_hh=0, s_x=0, s_hh=0, sm_x=1, sm_masked=masked,
                     pre=key_a + xfer, vring_state=ring_in, prefetch_v_hh=1)
        finish_phase(gen, f"{name}_a", 1, 1, 0)
        key_b = [I(f"s_lshl_b32 {sr(S_KEY0)}, {sr(S_J)}, 6"),
                 I(f"s_add_u32 {sr(S_KEY0)}, {sr(S_KEY0)}, 64")]
        # phase 2j+2: P.V(2j+1) (PB1, V half 1), S(2j+3) (SB1, K half 1), softmax(2j+2) (SB0)
        ring = phase(gen, pv_x=1, pv_hh=1, s_x=1, s_hh=1, sm_x=0, sm_masked=masked,
                     pre=key_b, vring_state=ring,
                     after_last_v=advance_slot(S_VSLOT, VVA, 8),
                     after_last_k=advance_slot(S_KSLOT, VKA, 8), prefetch_v_hh=0)
        finish_phase(gen, f"{name}_b", 0, 0, 1)
        # tile j + 2 (first read by the next iteration) has landed: the NSTAGE - 3 younger
        # tiles' transfers (8 instructions each) may still be in flight
        gen.emit([I(f"s_waitcnt vmcnt({(NSTAGE - 3) * 8})"), I("s_barrier")])
        lim = sr(S_JU) if not masked else sr(S_NM1)
        gen.emit([I(f"s_add_u32 {sr(S_J)}, {sr(S_J)}, 1"),
                  I(f"s_cmp_lt_u32 {sr(S_J)}, {lim}"),
                  I(f"s_cbranch_scc1 .L{name}")])
        lasts[masked] = gen.cur
        if not masked:
            gen.new_block("masked_check")
            gen.emit([I(".Lmasked_check:"),
                      I(f"s_cmp_ge_u32 {sr(S_J)}, {sr(S_NM1)}"),
                      I("s_cbranch_scc1 .Lepi")])
    b_mc = [b for b in gen.blocks if b.name == "masked_check"][0]
    firsts[False].preds = [pro_end, lasts[False]]
    b_mc.preds = [pro_end, lasts[False]]
    firsts[True].preds = [b_mc, lasts[True]]
    return [pro_end, b_mc, lasts[True]]


def iteration(gen: Gen, masked: bool, tag: str, jofs: int, ring_in, xfer_tile_ofs):
    """One loop iteration j = S_J + jofs (phases 2j+1, 2j+2), optionally issuing the transfer of
    tile S_J + xfer_tile_ofs at its start. Returns the V ring state after it."""
    xfer = []
    groups = []
    if xfer_tile_ofs is not None and not PAGED:
        # resources and stage first; the 8 transfer instructions spread over the phase's MFMAs
        xfer = [I(f"s_add_u32 {sr(S_TT)}, {sr(S_J)}, {xfer_tile_ofs}")] + \
            transfer_setup(sr(S_TT)) + \
            [I(f"s_add_u32 {sr(S_TSLOT)}, {sr(S_TSLOT)}, 1"),
             I(f"s_cmp_eq_u32 {sr(S_TSLOT)}, {NSTAGE}"),
             I(f"s_cselect_b32 {sr(S_TSLOT)}, 0, {sr(S_TSLOT)}")]
        assert not PREC
        # one load per group, each block's M0 write with its first load
        groups = []
        for which in ("k", "v"):
            tb = transfer_block(which)
            groups += [tb[:2]] + [[x] for x in tb[2:]]
    elif xfer_tile_ofs is not None:
        if PAGED:
            # tile j+3 from page-id lanes 0..3, tile j+4 from lanes 4..7; after the second's
            # page ids are read, the page ids of tiles j+5 and j+6 (waited for by the pair's
            # closing vmcnt(0)); the 8 transfer instructions spread over the phase's MFMAs
            assert PAIR and xfer_tile_ofs in (3, 4)
            body = transfer_paged(sr(S_TT), 4 * (xfer_tile_ofs - 3))
            nl = len(paged_loads())
            body, tb = body[:-nl], body[-nl:]
            groups = [tb[:2]] + [[x] for x in tb[2:5]] + [tb[5:7]] + [[x] for x in tb[7:]]
            if xfer_tile_ofs == 4:
                body += [I(f"s_add_u32 {sr(S_TT)}, {sr(S_J)}, 5")] + pt_load(sr(S_TT))
        else:
            body = transfer_setup(sr(S_TT)) + kv_transfers()
        xfer = [I(f"s_add_u32 {sr(S_TT)}, {sr(S_J)}, {xfer_tile_ofs}")] + body + \
            [I(f"s_add_u32 {sr(S_TSLOT)}, {sr(S_TSLOT)}, 1"),
             I(f"s_cmp_eq_u32 {sr(S_TSLOT)}, {NSTAGE}"),
             I(f"s_cselect_b32 {sr(S_TSLOT)}, 0, {sr(S_TSLOT)}")]
    key_a = [I(f"s_lshl_b32 {sr(S_KEY0)}, {sr(S_J)}, 6"),
             I(f"s_add_u32 {sr(S_KEY0)}, {sr(S_KEY0)}, {64 * jofs + 32}")]
    ring = phase(gen, pv_x=0, pv_hh=0, s_x=0, s_hh=0, sm_x=1, sm_masked=masked,
                 pre=key_a + xfer, vring_state=ring_in, prefetch_v_hh=1, spread=groups)
    finish_phase(gen, f"{tag}_a", 1, 1, 0)
    key_b = [I(f"s_lshl_b32 {sr(S_KEY0)}, {sr(S_J)}, 6"),
             I(f"s_add_u32 {sr(S_KEY0)}, {sr(S_KEY0)}, {64 * jofs + 64}")]
    ring = phase(gen, pv_x=1, pv_hh=1, s_x=1, s_hh=1, sm_x=0, sm_masked=masked,
                 pre=key_b, vring_state=ring,
                 after_last_v=advance_slot(S_VSLOT, VVA, 8),
                 after_last_k=advance_slot(S_KSLOT, VKA, 8), prefetch_v_hh=0)
    finish_phase(gen, f"{tag}_b", 0, 0, 1)
    return ring


def ring_entry(gen: Gen):
    pre_ids = list(range(gen.ds_next, gen.ds_next + 2 * RV))
    gen.ds_next += 2 * RV
    gen.ds_outstanding = list(pre_ids)
    return {"ready": {o: pre_ids[2 * o:2 * o + 2] for o in range(RV)}}


def pair_loops(gen: Gen, pro_end: Block) -> list:
    """Iterations in pairs (j, j+1) with one barrier per pair: the pair issues the transfers of
    tiles j+3 and j+4 (into the stages of tiles j-2 and j-1, dead since the previous barrier) and
    waits for both before its closing barrier; tiles j+2 .. j+4 are then resident for the next
    pair. Unmasked pairs while j + 2 <= JU, masked pairs while j + 2 <= n - 1, then at most one
    single (masked) iteration with no transfer (the tiles it reads landed by the last barrier)."""
    J, JU, NM1, T0 = sr(S_J), sr(S_JU), sr(S_NM1), sr(S_T0)
    gen.emit([I(f"s_mov_b32 {J}, 0")])
    blocks = {}
    for masked in (False, True):
        name = "pair_m" if masked else "pair_u"
        lim = NM1 if masked else JU
        chk = gen.new_block(f"{name}_check")
        blocks[f"{name}_check"] = chk
        gen.emit([I(f".L{name}_check:"),
                  I(f"s_add_u32 {T0}, {J}, 2"),
                  I(f"s_cmp_gt_u32 {T0}, {lim}"),
                  I(f"s_cbranch_scc1 .L{name}_done")])
        body = gen.new_block(name, [chk])
        blocks[name] = body
        ring = ring_entry(gen)
        ring = iteration(gen, masked, f"{name}0", 0, ring, 3)
        ring = iteration(gen, masked, f"{name}1", 1, ring, 4)
        gen.emit([I("s_waitcnt vmcnt(0)"), I("s_barrier"),
                  I(f"s_add_u32 {J}, {J}, 2"),
                  I(f"s_branch .L{name}_check")])
        blocks[f"{name}_end"] = gen.cur
        gen.new_block(f"{name}_done_blk")
        blocks[f"{name}_done_blk"] = gen.cur
        gen.emit(I(f".L{name}_done:"))
    # one single iteration when an odd number remains
    gen.emit([I(f"s_cmp_ge_u32 {J}, {NM1}"), I("s_cbranch_scc1 .Lepi")])
    single_chk = gen.cur
    sb = gen.new_block("single", [single_chk])
    ring = ring_entry(gen)
    iteration(gen, True, "single", 0, ring, None)
    single_end = gen.cur
    blocks["pair_u_check"].preds = [pro_end, blocks["pair_u_end"]]
    blocks["pair_u"].preds = [blocks["pair_u_check"]]
    blocks["pair_m_check"].preds = [blocks["pair_u_done_blk"], blocks["pair_m_end"]]
    blocks["pair_u_done_blk"].preds = [blocks["pair_u_check"]]
    blocks["pair_m"].preds = [blocks["pair_m_check"]]
    blocks["pair_m_done_blk"].preds = [blocks["pair_m_check"]]
    return [single_chk, single_end]


def finish_phase(gen: Gen, tag: str, x: int, hh: int, s_x) -> None:
    """End of a phase with a fast softmax: to the exact path when a row sum overflowed, then
    l += the half-tile's row sums."""
    gen.emit([I(f"s_cmp_lg_u64 {sr(S_MV, 2)}, 0"), I(f"s_cbranch_scc1 .Lexact_{tag}")])
    br = gen.cur
    cont = gen.new_block(f"cont_{tag}", [br])
    gen.emit(I(f".Lcont_{tag}:"))
    gen.emit([I(f"v_add_f32 {vr(V_L + rb)}, {vr(V_L + rb)}, {vr(V_LT + rb)}") for rb in range(2)])
    gen.exact.append((tag, x, hh, s_x, br, cont))


# --------------------------------------------------------------------------- output
def render_kernel(gen: Gen, name: str, num_vgpr: int = None, num_agpr: int = None,
                  num_sgpr: int = None, lds_bytes: int = None,
                  arg_bytes: int = None) -> tuple[list[str], list[str], list[str]]:
    """The text, kernel descriptor and metadata entry of one generated kernel (resource counts
    default to this generator's)."""
    NUM_VGPR = globals()["NUM_VGPR"] if num_vgpr is None else num_vgpr
    NUM_AGPR = globals()["NUM_AGPR"] if num_agpr is None else num_agpr
    NUM_SGPR = globals()["NUM_SGPR"] if num_sgpr is None else num_sgpr
    LDS_BYTES = globals()["LDS_BYTES"] if lds_bytes is None else lds_bytes
    ARG_BYTES = globals()["ARG_BYTES"] if arg_bytes is None else arg_bytes
    fix_hazards(gen.blocks)
    text = ["\t.text", f"\t.globl {name}", "\t.p2align 8", f"\t.type {name},@function", f"{name}:"]
    for b in gen.blocks:
        for x in b.ins:
            if x.kind == "nop":
                text.append("\t" + x.text)
                continue
            n = x.nops
            while n > 0:
                k = min(n, 16)
                text.append(f"\ts_nop {k - 1}")
                n -= k
            text.append(x.text if x.kind == "label" else "\t" + x.text)
    text += [".Lfunc_end:", f"\t.size {name}, .Lfunc_end-{name}", ""]
    acc_off = (NUM_VGPR + 3) // 4 * 4
    desc = ["\t.rodata", "\t.p2align 6", f"\t.amdhsa_kernel {name}",
            f"\t\t.amdhsa_group_segment_fixed_size {LDS_BYTES}",
            "\t\t.amdhsa_private_segment_fixed_size 0",
            f"\t\t.amdhsa_kernarg_size {ARG_BYTES}",
            "\t\t.amdhsa_user_sgpr_count 2",
            "\t\t.amdhsa_user_sgpr_kernarg_segment_ptr 1",
            "\t\t.amdhsa_system_sgpr_workgroup_id_x 1",
            "\t\t.amdhsa_system_vgpr_workitem_id 0",
            f"\t\t.amdhsa_next_free_vgpr {acc_off + NUM_AGPR}",
            f"\t\t.amdhsa_next_free_sgpr {NUM_SGPR}",
            f"\t\t.amdhsa_accum_offset {acc_off}",
            "\t\t.amdhsa_reserve_vcc 1",
            "\t\t.amdhsa_float_denorm_mode_32 3",
            "\t\t.amdhsa_float_denorm_mode_16_64 3",
            "\t\t.amdhsa_ieee_mode 1",
            "\t\t.amdhsa_dx10_clamp 1",
            "\t.end_amdhsa_kernel", ""]
    meta = [f"  - .agpr_count:     {NUM_AGPR}",
            "    .args:",
            "      - .offset:         0",
            f"        .size:           {ARG_BYTES}",
            "        .value_kind:     by_value",
            f"    .group_segment_fixed_size: {LDS_BYTES}",
            "    .kernarg_segment_align: 8",
            f"    .kernarg_segment_size: {ARG_BYTES}",
            "    .max_flat_workgroup_size: 256",
            f"    .name:           {name}",
            "    .private_segment_fixed_size: 0",
            f"    .sgpr_count:     {NUM_SGPR + 2}",
            f"    .symbol:         {name}.kd",
            f"    .vgpr_count:     {acc_off + NUM_AGPR}",
            "    .wavefront_size: 64"]
    return text, desc, meta


def render(kernels: list[tuple]) -> str:
    """One code object holding every kernel: (generator state, symbol, label prefix[, resource
    counts for render_kernel])."""
    lines = ['\t.amdgcn_target "amdgcn-amd-amdhsa--gfx950"', "\t.amdhsa_code_object_version 5"]
    metas = []
    for kern in kernels:
        gen, name, prefix = kern[:3]
        text, desc, meta = render_kernel(gen, name, **(kern[3] if len(kern) > 3 else {}))
        body = "\n".join(text + desc)
        if prefix:
            body = re.sub(r"\.L(\w+)", lambda m: f".L{prefix}{m.group(1)}", body)
        lines.append(body)
        metas += meta
    lines += ["\t.amdgpu_metadata", "---", "amdhsa.kernels:"] + metas + [
        "amdhsa.target:   amdgcn-amd-amdhsa--gfx950", "amdhsa.version:", "  - 1", "  - 2", "...",
        "\t.end_amdgpu_metadata"]
    return "\n".join(lines) + "\n"


def build_all() -> list[tuple]:
    """The contiguous, the paged and the precise kernel (with its resource counts: the precise
    kernel holds the Q residual in the last 64 AGPRs and three 48 KiB stages, one barrier per
    key tile)."""
    global PAGED, KERNEL, PREC, NSTAGE, PAIR, F16
    out = []
    for paged, prec, f16, name, prefix in ((False, False, False, KERNEL_CONTIG, ""),
                                           (True, False, False, KERNEL_PAGED, "P"),
                                           (False, True, False, KERNEL_PREC, "R"),
                                           (False, False, True, KERNEL_CONTIG_F16, "H"),
                                           (True, False, True, KERNEL_PAGED_F16, "HP")):
        PAGED, PREC, F16, KERNEL = paged, prec, f16, name
        NSTAGE, PAIR = (3, False) if prec else (5, True)
        counts = {"num_agpr": 256 if prec else NUM_AGPR,
                  "lds_bytes": NSTAGE * STAGE_BYTES()}
        out.append((build(), name, prefix, counts))
    PAGED, PREC, F16, KERNEL, NSTAGE, PAIR = False, False, False, KERNEL_CONTIG, 5, True
    return out


def fix_hazards_with_optional(blocks: list[Block]):
    """Hazard check over every path: block predecessors, plus inside a block the optional
    rescale sequences (between 's_cbranch_scc1 .Lnors_X' and '.Lnors_X:') taken or skipped."""
    def variants(seq: list[Ins]) -> list[list[Ins]]:
        out = [[]]
        i = 0
        while i < len(seq):
            x = seq[i]
            if x.text.startswith("s_cbranch_scc1 .Lnors_"):
                tag = x.text.split()[1]
                j = i + 1
                while not seq[j].text.startswith(tag + ":"):
                    j += 1
                opt = seq[i + 1:j]
                out = [v + [x] + opt for v in out] + [v + [x] for v in out]
                i = j
                continue
            out = [v + [x] for v in out]
            i += 1
        # cap the combinations: keep all-taken, all-skipped and single toggles
        return out[:8]

    for _ in range(3):
        for b in blocks:
            for t in tails(b):
                for v in variants(b.ins):
                    check_path(t + v, len(t))


def header(path: str):
    lines = ["// Generated by gen_prefill_a64.py: kernel-argument layout of fa_prefill_a64_bf16.",
             "#pragma once", f"#define FA_A64_ARG_BYTES {ARG_BYTES}",
             f"#define FA_A64_LDS_BYTES {LDS_BYTES}",
             f'#define FA_A64_KERNEL "{KERNEL_CONTIG}"',
             f'#define FA_A64_KERNEL_PAGED "{KERNEL_PAGED}"',
             f'#define FA_A64_KERNEL_PREC "{KERNEL_PREC}"',
             f'#define FA_A64_KERNEL_F16 "{KERNEL_CONTIG_F16}"',
             f'#define FA_A64_KERNEL_PAGED_F16 "{KERNEL_PAGED_F16}"']
    for n, off, sz in ARGS:
        lines.append(f"#define FA_A64_OFF_{n.upper()} {off}")
    open(path, "w").write("\n".join(lines) + "\n")


def blob(co_path: str, out_cpp: str):
    data = open(co_path, "rb").read()
    rows = [", ".join(f"0x{b:02x}" for b in data[i:i + 16]) for i in range(0, len(data), 16)]
    text = ("// Generated by gen_prefill_a64.py --blob: the assembled gfx950 code object of "
            "fa_prefill_a64_bf16.\n#include <stddef.h>\nnamespace fa {\n"
            f"extern const unsigned char kPrefillA64Co[] = {{\n" + ",\n".join(rows) +
            f"\n}};\nextern const size_t kPrefillA64CoSize = {len(data)};\n}}  // namespace fa\n")
    open(out_cpp, "w").write(text)


def main():
    if sys.argv[1] == "--blob":
        blob(sys.argv[2], sys.argv[3])
        return
    out_s, out_h = sys.argv[1], sys.argv[2]
    open(out_s, "w").write(render(build_all()))
    header(out_h)


if __name__ == "__main__":
    main()
