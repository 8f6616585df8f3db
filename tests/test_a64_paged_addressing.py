"""CPU check of the paged assembly prefill's address arithmetic (no GPU).

The generator (flat-attention_amd/csrc/gen_prefill_a64.py) emits the scalar code that turns a
block-table entry into the buffer resource of one 16-row page. A wrong base or bound there reads
outside the page pool, so this test executes the generated per-block set-up and the per-tile
transfer sequences in a small interpreter of the scalar instructions they use, for the cfg5
shape (8 sequences of 2560 keys in 16-row pages, shuffled tables) and ragged lengths, and checks
every transfer against the page it must read:
  * resource base = pool + kv_head * head bytes + page * 16 * row bytes (K and V),
  * resource bound = the page's live rows (kv_len - first key, clamped to 0..16) * row bytes,
  * a wave reads page `wave` of each 64-key tile (its rows 16 wave .. + 15), through one M0 per
    K or V block: M0 = stage * 32 KiB + 4 KiB * wave + (V: 16 KiB), instruction offsets
    1024 i for i = 0 .. 3 (LDS KiB 4 wave + i),
and every block-table load against the sequence's row (base, bound, first entry).
The same paths (pool row = page * 16 + in-page row) are what the reference's paged gather
reads (src/paged_kv.rs:113-174; oracle.paged_prefill)."""
import importlib.util
import os

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _gen():
    spec = importlib.util.spec_from_file_location(
        "gen_a64", os.path.join(ROOT, "flat-attention_amd", "csrc", "gen_prefill_a64.py"))
    g = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(g)
    return g


M32 = 0xFFFFFFFF


class Scalar:
    """SGPR file + the scalar/readlane subset the transfer code uses; records VMEM issues."""

    def __init__(self, g, pt):
        self.g = g
        self.s = {}
        self.scc = 0
        self.m0 = 0
        self.pt = pt          # page-id VGPR: lane -> value (set by the block-table loads)
        self.loads = []       # (kind, resource, m0 + instruction offset / soffset)

    def val(self, op):
        op = op.strip()
        if op.startswith("s") and op[1:].isdigit():
            return self.s.get(int(op[1:]), 0) & M32
        if op == "m0":
            return self.m0
        return int(op, 0) & M32

    def set(self, op, v):
        v &= M32
        if op == "m0":
            self.m0 = v
        else:
            self.s[int(op[1:])] = v

    def quad(self, op):  # "s[a:b]"
        a = int(op[2:op.index(":")])
        return [self.s.get(a + i, 0) & M32 for i in range(4)]

    def run(self, ins_list):
        for ins in ins_list:
            t = ins.text.strip()
            if not t or t.endswith(":"):
                continue
            op, _, rest = t.partition(" ")
            ops = [x.strip() for x in rest.split(",")]
            sx = lambda v: v - (1 << 32) if v & 0x80000000 else v  # noqa: E731
            if op == "s_mov_b32":
                self.set(ops[0], self.val(ops[1]))
            elif op == "s_add_u32":
                r = self.val(ops[1]) + self.val(ops[2])
                self.scc = r >> 32
                self.set(ops[0], r)
            elif op == "s_addc_u32":
                r = self.val(ops[1]) + self.val(ops[2]) + self.scc
                self.scc = r >> 32
                self.set(ops[0], r)
            elif op == "s_sub_u32":
                a, b = self.val(ops[1]), self.val(ops[2])
                self.scc = int(b > a)
                self.set(ops[0], a - b)
            elif op == "s_mul_i32":
                self.set(ops[0], self.val(ops[1]) * self.val(ops[2]))
            elif op == "s_mul_hi_u32":
                self.set(ops[0], (self.val(ops[1]) * self.val(ops[2])) >> 32)
            elif op == "s_lshl_b32":
                self.set(ops[0], self.val(ops[1]) << (self.val(ops[2]) & 31))
            elif op == "s_lshr_b32":
                self.set(ops[0], self.val(ops[1]) >> (self.val(ops[2]) & 31))
            elif op == "s_and_b32":
                self.set(ops[0], self.val(ops[1]) & self.val(ops[2]))
            elif op == "s_max_i32":
                self.set(ops[0], max(sx(self.val(ops[1])), sx(self.val(ops[2]))))
            elif op == "s_min_i32":
                self.set(ops[0], min(sx(self.val(ops[1])), sx(self.val(ops[2]))))
            elif op == "s_min_u32":
                self.set(ops[0], min(self.val(ops[1]), self.val(ops[2])))
            elif op == "s_max_u32":
                self.set(ops[0], max(self.val(ops[1]), self.val(ops[2])))
            elif op == "v_readlane_b32":
                self.set(ops[0], self.pt[self.val(ops[2])])
            elif op == "buffer_load_dwordx4" and rest.endswith("lds"):
                res = ops[1].split()[0]
                off = [int(w[7:]) for w in rest.split() if w.startswith("offset:")]
                self.loads.append(("xfer", self.quad(res), self.m0 + (off[0] if off else 0)))
            elif op == "buffer_load_dword":
                self.loads.append(("pt", self.quad(ops[2]), self.val(ops[3].split()[0])))
            elif op.startswith(("s_waitcnt", "s_nop")):
                continue
            else:
                raise AssertionError(f"unexpected instruction in the transfer code: {t}")


def _arg_sgpr(g, name, hi=False):
    return int(g.arg(name, hi)[1:])


def _setup_state(g, cpu, *, k_pool, v_pool, bt, bt_stride, kv_len, k_sh_bytes, row_bytes, b,
                 kvh, wave):
    """Argument SGPRs and the per-block registers the transfer code reads."""
    for name, v in (("k", k_pool), ("v", v_pool), ("bt", bt)):
        cpu.s[_arg_sgpr(g, name)] = v & M32
        cpu.s[_arg_sgpr(g, name, True)] = v >> 32
    cpu.s[_arg_sgpr(g, "k_sh")] = k_sh_bytes & M32
    cpu.s[_arg_sgpr(g, "k_sh", True)] = k_sh_bytes >> 32
    cpu.s[_arg_sgpr(g, "k_ss")] = row_bytes
    cpu.s[_arg_sgpr(g, "kv_len")] = kv_len
    cpu.s[_arg_sgpr(g, "bt_stride")] = bt_stride
    cpu.s[g.S_B] = b
    cpu.s[g.S_KVH] = kvh
    cpu.s[g.S_WAVE] = wave


def _paged_setup_block_ins(g):
    """The paged kernel's per-block set-up instructions (generator state of the paged build)."""
    g.PAGED, g.KERNEL = True, g.KERNEL_PAGED
    try:
        gen = g.build()
    finally:
        g.PAGED, g.KERNEL = False, g.KERNEL_CONTIG
    for blk in gen.blocks:
        if blk.name == "setup_block":
            return blk.ins
    raise AssertionError("no setup_block")


def _keep_transfer_code(ins_list, g):
    """From the set-up: the K/V base computation, block-table resource and loads, transfers.
    (Other scalar code, e.g. tile counts and the rotation, is not interpreted.)"""
    keep = []
    started = False
    for ins in ins_list:
        t = ins.text.strip()
        if t.startswith(".Lbatch_ok"):
            started = True
            continue
        if not started:
            continue
        if t.startswith(".Lq_norope") or t.startswith("s_cmp_eq_u32") and "rope_q" in t:
            break
        op = t.split(" ")[0]
        if op.startswith("v_") and op != "v_readlane_b32":
            continue
        if op.startswith(("s_cmp", "s_cselect", "s_cbranch", "s_branch", "s_barrier",
                          "s_endpgm", "s_bitcmp")):
            continue
        if op == "buffer_load_dwordx4" and not t.endswith("lds"):
            continue  # the Q loads
        keep.append(ins)
    return keep


def _expected_page(bt_row, kv_len, tile, wave):
    """(page id, live rows) of page `wave` of the tile."""
    key = 64 * tile + 16 * wave
    return (int(bt_row[key // 16]) if key < kv_len else None, max(0, min(16, kv_len - key)))


def _check_tile(loads, tile, stage, wave, page_rows, *, k_pool, v_pool, kvh_off, row_bytes):
    assert len(loads) == 8, loads
    page, rows = page_rows
    for j, (kind, res, lds) in enumerate(loads):
        which, i = ("k" if j < 4 else "v"), j % 4
        assert kind == "xfer"
        base = res[0] | ((res[1] & 0xFFFF) << 32)
        assert res[2] == rows * row_bytes, (tile, i, which, res[2], rows)
        assert res[3] == 0x20000
        if rows:
            pool = k_pool if which == "k" else v_pool
            assert base == pool + kvh_off + page * 16 * row_bytes, (tile, i, which)
        region = 0 if which == "k" else 16384
        assert lds == stage * 32768 + wave * 4096 + region + 1024 * i, (tile, i, which, lds)


@pytest.mark.parametrize("kv_len", [2560, 2553, 77, 16, 1])
@pytest.mark.parametrize("b,kvh,wave", [(0, 0, 0), (7, 5, 3), (3, 7, 1)])
def test_paged_transfers_read_exactly_their_pages(kv_len, b, kvh, wave):
    g = _gen()
    n_seq, hkv, D, ps = 8, 8, 128, 16
    row_bytes = hkv * D * 2
    bt_stride = (kv_len + ps - 1) // ps + 3   # wider rows than the sequence needs
    rng = np.random.default_rng(kv_len + 31 * b)
    bt = rng.permutation(n_seq * bt_stride).astype(np.int64).reshape(n_seq, bt_stride)
    k_pool, v_pool, bt_ptr = 0x7F1200000000, 0x7F5600001000, 0x7F9A00002000
    kw = dict(k_pool=k_pool, v_pool=v_pool, bt=bt_ptr, bt_stride=bt_stride, kv_len=kv_len,
              k_sh_bytes=D * 2, row_bytes=row_bytes, b=b, kvh=kvh, wave=wave)

    def table_slice(soffset):  # what a block-table load returns per lane (0 past the row)
        first = soffset // 4
        return [int(bt[b, first + l]) if first + l < bt_stride else 0 for l in range(64)]

    # ---- the per-block set-up: bases, block-table loads, transfers of tiles 0 .. 2
    cpu = Scalar(g, pt=[0] * 64)
    _setup_state(g, cpu, **kw)
    ins = _keep_transfer_code(_paged_setup_block_ins(g), g)
    # execute, serving each block-table load before the transfers that read it
    pending = []
    for x in ins:
        n = len(cpu.loads)
        cpu.run([x])
        if len(cpu.loads) > n and cpu.loads[-1][0] == "pt":
            kind, res, soff = cpu.loads[-1]
            base = res[0] | ((res[1] & 0xFFFF) << 32)
            assert base == bt_ptr + b * bt_stride * 4 and res[2] == bt_stride * 4
            pending.append(soff)
            if len(pending) == 1:
                cpu.pt = table_slice(soff)   # tiles 0 .. 2 read these
    xfers = [ld for ld in cpu.loads if ld[0] == "xfer"]
    assert pending == [0, 3 * 16], pending   # tiles 0..2, then tiles 3 and 4
    assert len(xfers) == 24
    kvh_off = kvh * D * 2
    for t in range(3):
        _check_tile(xfers[8 * t:8 * t + 8], t, t, wave, _expected_page(bt[b], kv_len, t, wave),
                    k_pool=k_pool, v_pool=v_pool, kvh_off=kvh_off, row_bytes=row_bytes)

    # ---- the loop: pair j transfers tiles j+3 (lanes 0..3) and j+4 (lanes 4..7) into the ring
    # stages, then loads the page ids of tiles j+5, j+6
    cpu.pt = table_slice(pending[1])
    tslot = 3
    n_tiles = max(1, (kv_len + 63) // 64) + 4
    for j in range(0, n_tiles, 2):
        for ofs in (3, 4):
            cpu.loads = []
            cpu.s[g.S_J] = j
            cpu.s[g.S_TSLOT] = tslot
            cpu.s[g.S_TT] = j + ofs
            body = g.transfer_paged(g.sr(g.S_TT), 4 * (ofs - 3))
            if ofs == 4:
                body += [g.I(f"s_add_u32 {g.sr(g.S_TT)}, {g.sr(g.S_J)}, 5")] + g.pt_load(g.sr(g.S_TT))
            cpu.run(body)
            _check_tile(cpu.loads[:8], j + ofs, tslot, wave,
                        _expected_page(bt[b], kv_len, j + ofs, wave),
                        k_pool=k_pool, v_pool=v_pool, kvh_off=kvh_off, row_bytes=row_bytes)
            if ofs == 4:
                kind, res, soff = cpu.loads[8]
                assert kind == "pt" and soff == (j + 5) * 16
                next_pt = table_slice(soff)
            tslot = (tslot + 1) % g.NSTAGE
        cpu.pt = next_pt
