"""CPU check of the assembly prefill's persistent block order (no GPU).

The generated per-block set-up (flat-attention_amd/csrc/gen_prefill_a64.py, setup_block) turns
(workgroup id, round) into the block (unit = (batch, kv head), query block) the workgroup runs
next, or ends the workgroup. This test executes exactly those generated scalar instructions, with
their branches, in a small interpreter, for every workgroup and round of several launch shapes,
and checks that:
  * every (unit, query block) of the launch is run exactly once, and every workgroup ends;
  * each round deals blocks heaviest first (query blocks in descending order over the list);
  * the causal work per workgroup stays balanced (the snake order pairs heavy with light).
The blocks' work is what the prefill computes for them (the reference's forward_reference
src/lib.rs:454-520 over rows qb*256 .. +255 of the grouped layout)."""
import importlib.util
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
M32 = 0xFFFFFFFF


def _gen():
    spec = importlib.util.spec_from_file_location(
        "gen_a64_order", os.path.join(ROOT, "flat-attention_amd", "csrc", "gen_prefill_a64.py"))
    g = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(g)
    return g


def _order_code(g):
    """setup_block's instructions from its first one up to the query-block computation."""
    gen = g.Gen()
    gen.exact = []
    b = gen.new_block("setup")
    g.setup(gen)
    gen.new_block("setup_block", [b])
    g.setup_block(gen)
    ins = [x.text.strip() for x in gen.cur.ins]
    end = next(i for i, t in enumerate(ins) if t.startswith(f"s_sub_u32 s{g.S_QB}, s{g.S_QB}"))
    return ins[:end + 1]


class Scalar:
    def __init__(self):
        self.s = {}
        self.scc = 0

    def val(self, op):
        if op.startswith("s") and op[1:].isdigit():
            return self.s.get(int(op[1:]), 0) & M32
        return int(op, 0) & M32

    def set(self, op, v):
        self.s[int(op[1:])] = v & M32

    def run(self, code):
        labels = {t[:-1]: i for i, t in enumerate(code) if t.endswith(":")}
        pc, steps = 0, 0
        while pc < len(code):
            steps += 1
            assert steps < 100000, "no exit"
            t = code[pc]
            pc += 1
            if t.endswith(":") or t.startswith(("s_barrier", "s_waitcnt", "s_nop")):
                continue
            op, _, rest = t.partition(" ")
            o = [x.strip() for x in rest.split(",")]
            if op == "s_endpgm":
                return None
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
            elif op == "s_sub_u32":
                a, b = self.val(o[1]), self.val(o[2])
                self.scc = int(b > a)
                self.set(o[0], a - b)
            elif op == "s_mul_i32":
                self.set(o[0], self.val(o[1]) * self.val(o[2]))
            elif op == "s_mul_hi_u32":
                self.set(o[0], (self.val(o[1]) * self.val(o[2])) >> 32)
            elif op == "s_lshr_b32":
                self.set(o[0], self.val(o[1]) >> (self.val(o[2]) & 31))
            elif op == "s_lshl_b32":
                self.set(o[0], self.val(o[1]) << (self.val(o[2]) & 31))
            elif op == "s_and_b32":
                r = self.val(o[1]) & self.val(o[2])
                self.scc = int(r != 0)
                self.set(o[0], r)
            elif op == "s_or_b32":
                r = self.val(o[1]) | self.val(o[2])
                self.scc = int(r != 0)
                self.set(o[0], r)
            elif op == "s_bitcmp1_b32":
                self.scc = (self.val(o[0]) >> self.val(o[1])) & 1
            elif op == "s_cselect_b32":
                self.set(o[0], self.val(o[1]) if self.scc else self.val(o[2]))
            elif op.startswith("s_cmp_"):
                a, b = self.val(o[0]), self.val(o[1])
                self.scc = int({"eq": a == b, "lg": a != b, "lt": a < b, "ge": a >= b,
                                "gt": a > b, "le": a <= b}[op.split("_")[2]])
            else:
                raise AssertionError(f"unexpected instruction in the block order: {t}")
        return True


def _fastdiv(d):
    sh = 0
    while (1 << sh) < d:
        sh += 1
    return ((1 << 32) * ((1 << sh) - d)) // d + 1, sh


def _schedule(g, code, units, nqb, grid):
    """(workgroup -> list of (unit, query block)) by running the generated code."""
    m, sh = _fastdiv(units)
    out = {}
    for w in range(grid):
        seq = []
        for rnd in range(10 * nqb + 10):
            cpu = Scalar()
            a = lambda n: int(g.arg(n)[1:])  # noqa: E731
            for n, v in (("units", units), ("nqb", nqb), ("nb", units * nqb), ("grid", grid),
                         ("fd_units_m", m), ("fd_units_s", sh)):
                cpu.s[a(n)] = v
            cpu.s[2] = w
            cpu.s[g.S_ROUND] = rnd
            if cpu.run(code) is None:
                break
            seq.append((cpu.s[g.S_BH], cpu.s[g.S_QB]))
        else:
            raise AssertionError("workgroup never ends")
        out[w] = seq
    return out


@pytest.mark.parametrize("units,nqb,grid", [
    (16, 64, 256),   # the cfg3 bench shape: B2 Hkv8, N4096 x group 4 / 256 rows
    (8, 40, 256),    # cfg5-like: 8 units
    (16, 64, 128),   # fewer workgroups
    (24, 7, 64),     # ragged rounds
    (5, 9, 13),      # units and grid off the XCD count
    (16, 3, 256),    # more workgroups than blocks
])
def test_every_block_once_heaviest_first(units, nqb, grid):
    g = _gen()
    code = _order_code(g)
    sched = _schedule(g, code, units, nqb, grid)
    seen = [b for seq in sched.values() for b in seq]
    assert sorted(seen) == sorted((u, q) for u in range(units) for q in range(nqb))
    # heaviest first: the blocks dealt in round r are never heavier than those of round r - 1
    rounds = max(len(s) for s in sched.values())
    for r in range(1, rounds):
        prev = [s[r - 1] for s in sched.values() if len(s) > r - 1]
        cur = [s[r] for s in sched.values() if len(s) > r]
        assert min(q for _, q in prev) >= max(q for _, q in cur), r


def test_causal_work_is_balanced_at_the_bench_shape():
    """cfg3 (16 units of 64 query blocks on 256 workgroups, four rounds): the snake order gives
    every workgroup the same causal work (query block qb needs qb + 1 key tiles of 256 rows)."""
    g = _gen()
    code = _order_code(g)
    sched = _schedule(g, code, 16, 64, 256)
    work = {w: sum(q + 1 for _, q in seq) for w, seq in sched.items()}
    assert len(set(work.values())) == 1, work
