"""CPU check of the assembly dK/dV kernel's address arithmetic (no GPU).

flat-attention_amd/csrc/gen_bwd_a64.py generates fa_bwd_dkdv_a64_bf16. Every global access it
makes goes through a buffer resource built by scalar code (base and byte range), plus an LDS
destination (M0) for the tile transfers. This test runs the generated program's scalar
instructions, with their branches, in a small interpreter for every workgroup and wave of
several launch shapes (vector, LDS and matrix instructions are skipped: they do not feed the
scalar addresses), and checks each access against the layout the HIP kernel bwd_dkdv<bf16, 128,
DMA, stored dS> uses (csrc/backward.hip; BackwardArgs in csrc/kernels.hpp):
  * the tiles a workgroup sweeps are every (head of the group, 128-query tile) its keys see
    (causal: the tiles from the key block's diagonal on), each once;
  * K / V: rows (batch, kv head) * seq + k0 .. + 31, 8 KiB; dK / dV stores the same rows;
  * the transfer of every tile after the first is issued during the tile before it, into the
    other LDS stage: Q and dO rows of (batch, group head) at the tile, 32 KiB, instruction i of
    wave w landing at LDS KiB 8 w + i (M0 per four instructions, instruction offsets 1 KiB apart,
    soffset 4 KiB for i >= 4); the bias rows (-LSE / scale then -delta,
    rows * 4 bytes further) by wave 0 into stage + 64 KiB, no bytes for waves 1..3;
  * the dS stores of every active 32-query sub-block at the group offset of
    ((b Hq + kvh G + hh) gph + base(t) + k0 / 32) * 8 KiB + 2 KiB * sub-block (base(t) =
    causal ? 2 t (t + 1) : t nb, gph the groups per head), bounded by the workspace;
  * nothing is transferred past the last tile (zero-byte resources).
The reference's backward (backward_reference_grouped src/backward_grouped.rs:17-95) fixes what
the products compute; this test pins where the kernel reads and writes them."""
import importlib.util
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
M32 = 0xFFFFFFFF


def _gen():
    spec = importlib.util.spec_from_file_location(
        "gen_bwd_a64_t", os.path.join(ROOT, "flat-attention_amd", "csrc", "gen_bwd_a64.py"))
    g = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(g)
    return g


def _program(g):
    gen = g.build()
    return [x.text.strip() for b in gen.blocks for x in b.ins]


class Scalar:
    def __init__(self):
        self.s = {}
        self.scc = 0
        self.m0 = 0
        self.events = []

    def val(self, op):
        op = op.strip()
        if op == "m0":
            return self.m0
        if op.startswith("s") and op[1:].isdigit():
            return self.s.get(int(op[1:]), 0) & M32
        return int(op, 0) & M32

    def set(self, op, v):
        if op == "m0":
            self.m0 = v & M32
        else:
            self.s[int(op[1:])] = v & M32

    def quad(self, op):
        a = int(op[2:op.index(":")])
        w = [self.s.get(a + i, 0) & M32 for i in range(4)]
        return (w[0] | ((w[1] & 0xFFFF) << 32), w[2])

    def run(self, code):
        labels = {t[:-1]: i for i, t in enumerate(code) if t.endswith(":")}
        pc = steps = 0
        while pc < len(code):
            steps += 1
            assert steps < 2_000_000
            t = code[pc]
            pc += 1
            if not t or t.endswith(":"):
                continue
            op, _, rest = t.partition(" ")
            o = [x.strip() for x in rest.split(",")]
            if op == "s_endpgm":
                return
            if op.startswith(("v_", "ds_", "s_waitcnt", "s_nop", "s_barrier", "s_load")):
                continue
            if op == "s_branch":
                pc = labels[o[0]]
            elif op == "s_cbranch_scc0":
                pc = labels[o[0]] if self.scc == 0 else pc
            elif op == "s_cbranch_scc1":
                pc = labels[o[0]] if self.scc == 1 else pc
            elif op == "s_mov_b32":
                self.set(o[0], self.val(o[1]))
            elif op == "s_add_u32":
                r = self.val(o[1]) + self.val(o[2])
                self.scc = r >> 32
                self.set(o[0], r)
            elif op == "s_addc_u32":
                r = self.val(o[1]) + self.val(o[2]) + self.scc
                self.scc = r >> 32
                self.set(o[0], r)
            elif op == "s_sub_u32":
                a, b = self.val(o[1]), self.val(o[2])
                self.scc = int(b > a)
                self.set(o[0], a - b)
            elif op == "s_mul_i32":
                self.set(o[0], self.val(o[1]) * self.val(o[2]))
            elif op == "s_mul_hi_u32":
                self.set(o[0], (self.val(o[1]) * self.val(o[2])) >> 32)
            elif op == "s_lshl_b32":
                r = self.val(o[1]) << (self.val(o[2]) & 31)
                self.scc = int((r & M32) != 0)
                self.set(o[0], r)
            elif op == "s_lshr_b32":
                r = self.val(o[1]) >> (self.val(o[2]) & 31)
                self.scc = int(r != 0)
                self.set(o[0], r)
            elif op == "s_and_b32":
                r = self.val(o[1]) & self.val(o[2])
                self.scc = int(r != 0)
                self.set(o[0], r)
            elif op == "s_cselect_b32":
                self.set(o[0], self.val(o[1]) if self.scc else self.val(o[2]))
            elif op.startswith("s_cmp_"):
                a, b = self.val(o[0]), self.val(o[1])
                self.scc = int({"eq": a == b, "lg": a != b, "lt": a < b, "ge": a >= b,
                                "gt": a > b, "le": a <= b}[op.split("_")[2]])
            elif op == "buffer_load_dwordx4" and rest.endswith(" lds"):
                res = self.quad(o[1])
                soff = self.val(o[2].split()[0])
                off = int(rest.split("offset:")[1].split()[0]) if "offset:" in rest else 0
                self.events.append(("xfer", res, soff, self.m0 + off, t))
            elif op == "buffer_load_dwordx4":
                off = int(rest.split("offset:")[1]) if "offset:" in rest else 0
                self.events.append(("load", self.quad(o[2]), off, None, t))
            elif op == "buffer_store_dwordx4":
                soff = self.val(o[3].split()[0])
                off = int(rest.split("offset:")[1].split()[0]) if "offset:" in rest else 0
                self.events.append(("store", self.quad(o[2]), soff + off, None, t))
            else:
                raise AssertionError(f"unexpected scalar instruction: {t}")
        raise AssertionError("fell off the program")


def _fastdiv(d):
    sh = 0
    while (1 << sh) < d:
        sh += 1
    return ((1 << 32) * ((1 << sh) - d)) // d + 1, sh


BASE = {"q": 0x10_0000_0000, "k": 0x20_0000_0000, "v": 0x30_0000_0000, "dout": 0x40_0000_0000,
        "dk": 0x50_0000_0000, "dv": 0x60_0000_0000, "ld": 0x70_0000_0000, "ds": 0x80_0000_0000}


def _args(g, B, Hq, Hkv, S, causal):
    G = Hq // Hkv
    nbk = B * Hkv
    nt = S // 128
    nb = (S + 31) // 32
    gph = 2 * nt * (nt + 1) if causal else nt * nb
    ds_bytes = B * Hq * gph * 8192
    a = dict(seq=S, group=G, q_heads=Hq, kv_heads=Hkv, causal=int(causal), c2=0, scale=0,
             ds_nb=nb, ds_gph=gph, ds_bytes=ds_bytes, nbk=nbk, rows=B * Hq * S)
    a["fd_nbk_m"], a["fd_nbk_s"] = _fastdiv(nbk)
    a["fd_kvh_m"], a["fd_kvh_s"] = _fastdiv(Hkv)
    return a, gph, nb, ds_bytes


def _run_wave(g, code, args, bid, w):
    cpu = Scalar()
    for name, off, sz in g.ARGS:
        v = BASE[name] if name in BASE else args[name]
        cpu.s[g.ARG_SGPR0 + off // 4] = v & M32
        if sz == 8:
            cpu.s[g.ARG_SGPR0 + off // 4 + 1] = v >> 32
    cpu.s[2] = bid
    cpu.s[g.S_WAVE] = 64 * w          # v_readfirstlane of the thread id of lane 0
    cpu.run(code)
    return cpu.events


SHAPES = [(1, 4, 1, 256, True), (2, 8, 2, 384, True), (2, 8, 2, 384, False),
          (1, 2, 2, 512, True), (1, 16, 2, 256, False), (1, 1, 1, 128, True)]


@pytest.mark.parametrize("B,Hq,Hkv,S,causal", SHAPES)
def test_every_access_matches_the_layout(B, Hq, Hkv, S, causal):
    g = _gen()
    code = _program(g)
    args, gph, nb, ds_bytes = _args(g, B, Hq, Hkv, S, causal)
    G, nbk, RB = Hq // Hkv, B * Hkv, 256
    rows = B * Hq * S
    for bid in range(S // 128 * nbk):
        kb, bkv = bid // nbk, bid % nbk
        b, kvh = bkv // Hkv, bkv % Hkv
        qstart = 128 * kb if causal else 0
        want_tiles = {(hh, qt) for hh in range(G) for qt in range(qstart, S, 128)}
        for w in range(4):
            ev = _run_wave(g, code, args, bid, w)
            k0 = 128 * kb + 32 * w
            krow = (bkv * S + k0) * RB
            loads = [e for e in ev if e[0] == "load"]
            assert len(loads) == 16
            for i, (_, (base, nrec), off, _, t) in enumerate(loads):
                src = "k" if i < 8 else "v"
                assert (base, nrec, off) == (BASE[src] + krow, 32 * RB, 32 * (i % 8)), t
            # transfers: groups of 17 per tile (16 Q / dO + 1 bias)
            xf = [e for e in ev if e[0] == "xfer"]
            assert len(xf) % 17 == 0
            tiles = []
            for j in range(len(xf) // 17):
                grp = xf[17 * j:17 * j + 17]
                stage = (j % 2) * g.STAGE
                qbase, qn = grp[0][1]
                if qn == 0:          # past the last tile: nothing read
                    assert all(e[1][1] == 0 for e in grp), j
                    continue
                row0 = (qbase - BASE["q"]) // RB
                assert (qbase - BASE["q"]) % RB == 0
                head, qt = divmod(row0, S)
                bq, hq = divmod(head, Hq)
                assert bq == b and kvh * G <= hq < kvh * G + G, (bid, w, j)
                tiles.append((hq - kvh * G, qt))
                for i in range(8):
                    _, (base, n), soff, lds, t = grp[i]
                    assert (base, n, soff) == (qbase, 128 * RB, 4096 * (i // 4)), t
                    assert lds == stage + 8192 * w + 1024 * i, t
                    _, (base, n), soff, lds, t = grp[8 + i]
                    assert (base, n, soff) == (BASE["dout"] + row0 * RB, 128 * RB,
                                               4096 * (i // 4)), t
                    assert lds == stage + g.T_DO + 8192 * w + 1024 * i, t
                _, (base, n), soff, m0, t = grp[16]
                assert base == BASE["ld"] + 4 * row0 and soff == 0, t
                if w == 0:
                    assert (n, m0) == (4 * rows + 512, stage + g.T_LD), t
                else:
                    assert (n, m0) == (0, g.DUMMY), t
            assert len(tiles) == len(set(tiles)) and set(tiles) == want_tiles, (bid, w)
            # dS stores: every active sub-block of every tile
            st = [e for e in ev if e[0] == "store"][:-16]
            ds_seen = []
            for _, (base, n), off, _, t in st:
                goff = base - BASE["ds"]
                assert n == ds_bytes - goff, t
                assert 0 <= goff and goff + off + 1024 <= ds_bytes, t   # 64 lanes x 16 bytes
                ds_seen.append(goff + off)
            want = []
            for hh, qt in sorted(want_tiles):
                tix = qt // 128
                base_t = 2 * tix * (tix + 1) if causal else tix * nb
                goff = ((b * Hq + kvh * G + hh) * gph + base_t + k0 // 32) * 8192
                s0 = w if causal and qt == qstart else 0
                for sb in range(s0, 4):
                    want += [goff + 2048 * sb, goff + 2048 * sb + 1024]
            assert sorted(ds_seen) == sorted(want), (bid, w)
            # epilogue: dV then dK rows of the wave's keys, 1 KiB per store
            ep = [e for e in ev if e[0] == "store"][-16:]
            for i, (_, (base, n), off, _, t) in enumerate(ep):
                dst = "dv" if i < 8 else "dk"
                assert (base, n, off) == (BASE[dst] + krow, 32 * RB, 1024 * (i % 8)), t
