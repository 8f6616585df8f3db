"""CPU check of the assembly prefill's per-lane K/V transfer offsets (no GPU).

A K or V tile lands in LDS as 64 rows of 256 bytes whose 16-byte chunks are XOR-swizzled: slot s
of row r holds chunk s ^ swz(r), swz(r) = 4 (r & 3) + ((r >> 2) & 3), the layout the K and V^T
operand reads assume. Each wave moves its part of a tile with four `buffer_load_dwordx4 ... lds`
instructions that share one M0 (stage base + 4 KiB * wave) and differ in their instruction
offset 1024 i, which moves the LDS and the global address alike; the per-lane offsets VTOFF + i
carry the rest. This test executes the generated per-lane code that computes VTOFF (the
contiguous and the paged kernel, several row strides) lane by lane and checks, for every wave,
instruction and lane, that the global bytes a load reads are the row and chunk its LDS slot must
hold: tile row r (contiguous) or in-page row r - 16 wave of the wave's page (paged). The same for
the assembly backward's Q / dO transfers (gen_bwd_a64.py: 128-row tiles, instruction i of wave w
at LDS KiB 8 w + i, M0 + 4 KiB and soffset 4096 for i >= 4)."""
import importlib.util
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
M32 = 0xFFFFFFFF


def _gen(name="gen_prefill_a64"):
    spec = importlib.util.spec_from_file_location(
        f"{name}_xfer", os.path.join(ROOT, "flat-attention_amd", "csrc", f"{name}.py"))
    g = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(g)
    return g


def _offset_code(g, paged):
    """setup_block's instructions from the first one writing V_ROW from the lane id through
    the last write of VTOFF + 3."""
    g.PAGED, g.KERNEL = paged, (g.KERNEL_PAGED if paged else g.KERNEL_CONTIG)
    try:
        gen = g.build()
    finally:
        g.PAGED, g.KERNEL = False, g.KERNEL_CONTIG
    ins = next(b.ins for b in gen.blocks if b.name == "setup_block")
    texts = [x.text.strip() for x in ins]
    first = texts.index(f"v_lshrrev_b32 {g.vr(g.V_ROW)}, 4, {g.vr(g.V_LANE)}")
    last = max(i for i, t in enumerate(texts)
               if t.split(" ", 1)[0].startswith("v_") and
               t.split(" ", 1)[1].startswith(f"{g.vr(g.VTOFF + 3)},"))
    return texts[first:last + 1]


def _run(code, lane, sgpr):
    v = {}

    def val(op):
        op = op.strip()
        if op[0] in "vs" and op[1:].isdigit():
            return (v if op[0] == "v" else sgpr).get(int(op[1:]), 0) & M32
        return int(op, 0) & M32

    v[1] = lane  # V_LANE
    for t in code:
        op, _, rest = t.partition(" ")
        o = [x.strip() for x in rest.split(",")]
        d = int(o[0][1:])
        if op == "s_lshl_b32":
            sgpr[d] = (val(o[1]) << (val(o[2]) & 31)) & M32
            continue
        a = [val(x) for x in o[1:]]
        if op == "v_lshrrev_b32":
            r = a[1] >> (a[0] & 31)
        elif op == "v_lshlrev_b32":
            r = a[1] << (a[0] & 31)
        elif op == "v_and_b32":
            r = a[0] & a[1]
        elif op == "v_xor_b32":
            r = a[0] ^ a[1]
        elif op == "v_add_u32":
            r = a[0] + a[1]
        elif op == "v_mul_lo_u32":
            r = a[0] * a[1]
        elif op == "v_lshl_add_u32":
            r = (a[0] << (a[1] & 31)) + a[2]
        elif op == "v_mov_b32":
            r = a[0]
        else:
            raise AssertionError(f"unexpected instruction in the offset code: {t}")
        v[d] = r & M32
    return v


def _swz(r):
    return 4 * (r & 3) + ((r >> 2) & 3)


@pytest.mark.parametrize("paged", [False, True])
@pytest.mark.parametrize("row_bytes", [256, 2048, 4352])
def test_every_lane_reads_the_chunk_its_lds_slot_holds(paged, row_bytes):
    g = _gen()
    code = _offset_code(g, paged)
    seen = set()
    for wave in range(4):
        for lane in range(64):
            sgpr = {int(g.arg("k_ss")[1:]): row_bytes, g.S_WAVE: wave}
            v = _run(code, lane, sgpr)
            for i in range(4):
                voff = v[g.VTOFF + i]
                assert voff < 2 ** 31, (wave, lane, i)
                glob = voff + 1024 * i                       # bytes from the resource base
                lds = 4096 * wave + 1024 * i + 16 * lane     # bytes into the K (or V) region
                r, slot = lds // 256, (lds % 256) // 16
                row = r - 16 * wave if paged else r          # paged: the wave's page
                assert 0 <= row < (16 if paged else 64)
                assert glob // row_bytes == row, (wave, lane, i, glob)
                assert (glob % row_bytes) // 16 == slot ^ _swz(r), (wave, lane, i, glob)
                seen.add(lds)
    assert len(seen) == 1024  # the 16 KiB region exactly once


def test_backward_lanes_read_the_chunks_their_lds_slots_hold():
    g = _gen("gen_bwd_a64")
    texts = [x.text.strip() for b in g.build().blocks for x in b.ins]
    first = texts.index(f"v_lshrrev_b32 {g.vr(g.V_TMP + 3)}, 4, {g.vr(g.V_LANE)}")
    last = max(i for i, t in enumerate(texts)
               if t.startswith("v_") and t.split(" ", 1)[1].startswith(f"{g.vr(g.xoff(3))},"))
    code = texts[first:last + 1]
    seen = set()
    for wave in range(4):
        for lane in range(64):
            v = _run(code, lane, {g.S_WAVE: wave})
            for i in range(8):
                glob = v[g.xoff(i % 4)] + 1024 * (i % 4) + 4096 * (i // 4)
                lds = 8192 * wave + 1024 * i + 16 * lane
                r, slot = lds // 256, (lds % 256) // 16
                assert glob // 256 == r, (wave, lane, i, glob)
                assert (glob % 256) // 16 == slot ^ _swz(r), (wave, lane, i, glob)
                seen.add(lds)
    assert len(seen) == 2048  # the 32 KiB Q (or dO) tile exactly once
