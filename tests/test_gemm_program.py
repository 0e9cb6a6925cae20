"""The generated GEMM tile program (kernels/gen_gemm.py), checked on the CPU.

The whole-tile GEMM runs one inline-asm statement that the compiler only assembles
line by line, so what would otherwise show only on the GPU is checked here from the
program text:
- branches land on labels of the program, labels are unique, every register the
  program names is in its clobber set, m0 is saved on entry and restored at the exit;
- a walk of the scalar control flow for several K: the MFMA and DMA counts, and the
  LDS ring discipline.  Every wave runs the same program, so for each LDS buffer the
  walk checks that a fragment read sees a DMA fill that this wave waited for (vmcnt)
  before a barrier that precedes the read, and that a DMA into a buffer comes after a
  barrier that follows the completion (lgkmcnt) of the last read of it.  The SiLU*Mul
  program stages each wave's UP tile over the ring: its DMA must follow a barrier that
  comes after every ring read and every ring fill completed, and its reads must follow
  the wave's own wait for it.
"""
import re
import sys
from pathlib import Path

import pytest

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "tile-rs_amd" / "csrc" / "kernels"))
import gen_gemm as G  # noqa: E402

OP = G.OP
CLOBBER_V = set(range(16, 256))
CLOBBER_A = set(range(256))
CLOBBER_S = set(range(48, 58))
CLOBBER_S_SILU = set(range(48, 60))


def regs(text, kind):
    out = set()
    for a, b in re.findall(rf"\b{kind}\[(\d+):(\d+)\]", text):
        out |= set(range(int(a), int(b) + 1))
    out |= {int(a) for a in re.findall(rf"\b{kind}(\d+)\b", text)}
    return out


def static_problems(prog, sregs=CLOBBER_S):
    lines = [l.strip() for l in prog]
    defs = [l[:-1] for l in lines if l.endswith(":")]
    bad = [f"label defined twice: {d}" for d in set(defs) if defs.count(d) > 1]
    for ln in lines:
        if not ln or ln.endswith(":"):
            continue
        op, _, body = ln.partition(" ")
        if op.startswith("s_branch") or op.startswith("s_cbranch"):
            if body.strip() not in defs:
                bad.append("branch outside the program: " + ln)
        elif op.startswith("s_setpc") or op.startswith("s_swappc"):
            bad.append("unexpected control transfer: " + ln)
        if regs(body, "v") - CLOBBER_V:
            bad.append("VGPR outside the clobber list: " + ln)
        if regs(body, "a") - CLOBBER_A:
            bad.append("AGPR outside the clobber list: " + ln)
        if regs(body, "s") - sregs:
            bad.append("SGPR outside the clobber list: " + ln)
        for kind in ("v", "a"):
            for a, b in re.findall(rf"\b{kind}\[(\d+):(\d+)\]", body):
                if int(a) % 2:
                    bad.append("odd-aligned register tuple: " + ln)
    return bad


class Walk:
    """Scalar control flow of one wave, with the LDS buffer accounting."""

    def __init__(self, prog, nk, bt):
        self.prog = [l.strip() for l in prog]
        self.labels = {l[:-1]: i for i, l in enumerate(self.prog) if l.endswith(":")}
        self.ops = {OP["nk"]: nk}
        self.bt = bt
        self.s, self.scc, self.m0 = {}, 0, None
        self.vmem = []      # buffer tag of each vector memory op (None: a store)
        self.vm_done = 0    # prefix of self.vmem known complete
        self.lgkm = []      # buffer tag of each LDS read
        self.lgkm_done = 0
        self.t = 0          # instruction counter
        self.barriers = []  # times of the barriers
        self.fill = {}      # buffer -> (vmem index, issue time) of its latest DMA
        self.fill_done = {}  # buffer -> time its latest DMA was seen complete
        self.read = {}      # buffer -> (lgkm index, issue time) of its latest read
        self.read_done = {}  # buffer -> time its latest read was seen complete
        self.mfma = self.dma = self.stores = 0
        self.problems = []

    def val(self, tok):
        tok = tok.strip()
        if tok.startswith("%"):
            return self.ops.get(int(tok[1:]), 0)
        m = re.fullmatch(r"s\[(\d+):\d+\]", tok) or re.fullmatch(r"s(\d+)", tok)
        if m:
            return self.s.get(int(m.group(1)), 0)
        return int(tok, 0)

    def put(self, tok, v):
        m = re.fullmatch(r"s\[(\d+):\d+\]", tok) or re.fullmatch(r"s(\d+)", tok)
        assert m, tok
        self.s[int(m.group(1))] = v & 0xffffffff

    def a_buf(self, off):
        return ("A", off // 32768)

    def b_buf(self, off):
        return ("B", off // (32768 if self.bt else 16384))

    def barrier_between(self, t0, t1):
        return any(t0 <= b < t1 for b in self.barriers)

    def on_read(self, buf):
        f = self.fill.get(buf)
        if f is None:
            self.problems.append(f"read of {buf} never filled (t={self.t})")
        else:
            done = self.fill_done.get(buf)
            if done is None or done < f[1] or not self.barrier_between(done, self.t):
                self.problems.append(f"read of {buf} at t={self.t} before its fill is waited and synced")
        self.lgkm.append(buf)
        self.read[buf] = (len(self.lgkm) - 1, self.t)

    def on_up_dma(self):
        for buf, (_, t) in self.read.items():
            done = self.read_done.get(buf)
            if done is None or done < t or not self.barrier_between(done, self.t):
                self.problems.append(f"UP staging at t={self.t} over {buf} before its reads are done and synced")
        for buf, (_, t) in self.fill.items():
            if buf[0] == "U":
                continue
            done = self.fill_done.get(buf)
            if done is None or done < t or not self.barrier_between(done, self.t):
                self.problems.append(f"UP staging at t={self.t} over {buf} before its fill is done and synced")
        self.vmem.append(("U", 0))
        self.fill[("U", 0)] = (len(self.vmem) - 1, self.t)
        self.dma += 1

    def on_up_read(self):
        f = self.fill.get(("U", 0))
        done = self.fill_done.get(("U", 0))
        if f is None or done is None or done < f[1]:
            self.problems.append(f"UP read at t={self.t} before the wave's own UP DMA is waited")

    def on_dma(self, buf):
        r = self.read.get(buf)
        if r is not None:
            done = self.read_done.get(buf)
            if done is None or done < r[1] or not self.barrier_between(done, self.t):
                self.problems.append(f"DMA into {buf} at t={self.t} before its last read is done and synced")
        self.vmem.append(buf)
        self.fill[buf] = (len(self.vmem) - 1, self.t)
        self.dma += 1

    def run(self, limit=1_000_000):
        pc = 0
        while pc < len(self.prog):
            self.t += 1
            assert self.t < limit, "no exit"
            line = self.prog[pc]
            pc += 1
            if not line or line.endswith(":"):
                continue
            op, _, rest = line.partition(" ")
            a = [x.strip() for x in rest.split(",")] if rest else []
            if op == "global_load_lds_dwordx4":
                kind, imm = self.m0
                if kind == "U":
                    self.on_up_dma()
                else:
                    self.on_dma(self.a_buf(imm) if kind == "A" else self.b_buf(imm))
            elif op == "ds_read_u16":
                assert a[1].split()[0] == f"%{OP['uread']}", line
                self.on_up_read()
            elif op.startswith("global_store"):
                self.vmem.append(None)
                self.stores += 1
            elif op.startswith("ds_read"):
                base = int(re.match(r"v(\d+)", a[1]).group(1))
                off = int(re.search(r"offset:(\d+)", rest).group(1)) if "offset:" in rest else 0
                self.on_read(self.a_buf(off) if base in G.VA else self.b_buf(off))
            elif op.startswith("v_mfma"):
                self.mfma += 1
            elif op == "s_waitcnt":
                m = re.search(r"vmcnt\((\d+)\)", rest)
                if m:
                    self.vm_done = max(self.vm_done, len(self.vmem) - int(m.group(1)))
                    for buf, (i, _) in self.fill.items():
                        if i < self.vm_done and self.fill_done.get(buf, -1) < self.fill[buf][1]:
                            self.fill_done[buf] = self.t
                m = re.search(r"lgkmcnt\((\d+)\)", rest)
                if m:
                    self.lgkm_done = max(self.lgkm_done, len(self.lgkm) - int(m.group(1)))
                    for buf, (i, _) in self.read.items():
                        if i < self.lgkm_done and self.read_done.get(buf, -1) < self.read[buf][1]:
                            self.read_done[buf] = self.t
            elif op == "s_barrier":
                self.barriers.append(self.t)
            elif op.startswith("v_") or op == "s_nop":
                pass
            elif op == "s_add_u32" and a[0] == "m0":
                kind = {f"%{OP['ldsa']}": "A", f"%{OP['ldsb']}": "B", f"%{OP['ustage']}": "U"}[a[1]]
                self.m0 = (kind, int(a[2], 0))
            elif op == "s_mov_b32" and "m0" in a:
                pass
            elif op in ("s_mov_b32", "s_mov_b64"):
                self.put(a[0], self.val(a[1]))
            elif op in ("s_add_u32", "s_addc_u32"):
                self.put(a[0], self.val(a[1]) + self.val(a[2]))
            elif op == "s_sub_u32":
                self.put(a[0], self.val(a[1]) - self.val(a[2]))
            elif op == "s_mul_i32":
                self.put(a[0], self.val(a[1]) * self.val(a[2]))
            elif op == "s_lshr_b32":
                self.put(a[0], self.val(a[1]) >> self.val(a[2]))
            elif op == "s_lshl_b32":
                self.put(a[0], self.val(a[1]) << self.val(a[2]))
            elif op.startswith("s_cmp_"):
                x, y = self.val(a[0]), self.val(a[1])
                self.scc = int({"eq": x == y, "lg": x != y}[op.split("_")[2]])
            elif op == "s_bitcmp1_b32":
                self.scc = (self.val(a[0]) >> self.val(a[1])) & 1
            elif op in ("s_cbranch_scc0", "s_cbranch_scc1", "s_branch"):
                if op == "s_branch" or self.scc == int(op[-1]):
                    pc = self.labels[a[0]]
            else:
                raise AssertionError("unmodelled instruction: " + line)
        return self


CASES = [(dt, out, bt) for dt in ("bf16", "f16") for out in ("f32", "bf16", "f16") for bt in (False, True)]


@pytest.mark.parametrize("dt,out,bt", CASES)
def test_program_text_is_self_contained(dt, out, bt):
    prog = G.program(dt, out, bt)
    assert static_problems(prog) == []
    assert prog[0] == "s_mov_b32 s55, m0" and prog[-1] == "s_mov_b32 m0, s55"
    assert not any("s55" in l for l in prog[1:-1])
    if out != "f32":
        silu = G.program(dt, out, bt, silu=True)
        assert static_problems(silu, CLOBBER_S_SILU) == []
        assert silu[0] == "s_mov_b32 s55, m0" and silu[-1] == "s_mov_b32 m0, s55"
        assert not any("s55" in l for l in silu[1:-1])


def test_clobber_lists_match_the_checked_sets():
    text = Path(G.__file__).read_text()
    assert "for k in range(16, 256)" in text and "for k in range(256)" in text
    assert "for k in range(48, 58)" in text and 'TH_GEMM_ASM_CLOBBERS, \\"s58\\", \\"s59\\"' in text


def test_static_check_finds_planted_cases():
    assert static_problems(["s_branch L_x_%="])
    assert static_problems(["L1:", "L1:"])
    assert static_problems(["v_mov_b32 v3, v40"])
    assert static_problems(["s_mov_b32 s60, s48"])
    assert static_problems(["ds_read_b128 v[129:132], v16"])
    assert not static_problems(["L1:", "s_cbranch_scc1 L1", "v_accvgpr_read_b32 v40, a255"])


@pytest.mark.parametrize("bt", [False, True])
@pytest.mark.parametrize("out", ["f32", "bf16"])
@pytest.mark.parametrize("nk", [8, 12, 16, 20, 36, 128])
def test_ring_discipline_and_counts(nk, out, bt):
    """K = 32 nk: every fragment read sees a waited, synchronized fill; no DMA overwrites
    a buffer before every wave is done reading it; one MFMA per 16x16 block and K step;
    every A and B row of the tile loaded once; the C tile stored once; no DMA left in
    flight at the exit."""
    w = Walk(G.program("bf16", out, bt), nk, bt).run()
    assert w.problems == []
    assert w.mfma == 64 * nk
    assert w.dma == 8 * nk          # A: 8 units per 64-k double stage; B: 4 per 32-k stage (8 per 64 with bt)
    assert w.stores == 256
    assert w.vm_done == len(w.vmem)


@pytest.mark.parametrize("bt", [False, True])
@pytest.mark.parametrize("nk", [8, 12, 128])
def test_silu_program_ring_discipline_and_counts(nk, bt):
    w = Walk(G.program("f16", "f16", bt, silu=True), nk, bt).run()
    assert w.problems == []
    assert w.mfma == 64 * nk
    assert w.dma == 8 * nk + 32      # the ring, then 32 UP units (128 rows x 256 B)
    assert w.stores == 256
    assert w.vm_done == len(w.vmem)


def test_walk_finds_a_planted_early_up_staging():
    """The UP staging needs the barrier that opens the last step: without it a slower
    wave may still read its last fragments where this wave's UP lands."""
    prog = G.program("f16", "f16", False, silu=True)
    i = max(k for k, l in enumerate(prog) if l == "s_barrier")
    assert Walk(prog[:i] + prog[i + 1:], 16, False).run().problems


def test_walk_finds_a_planted_race():
    """Drop the barrier of one steady-state step: the walk must report the buffer that
    the next DMA overwrites while other waves may still read it."""
    prog = G.program("bf16", "f32", False)
    top = prog.index("L_top_%=:")
    i = prog.index("s_barrier", top)
    planted = prog[:i] + prog[i + 1:]
    assert Walk(planted, 16, False).run().problems
    assert Walk(prog, 16, False).run().problems == []


@pytest.mark.parametrize("bt", [False, True])
def test_walk_finds_planted_wait_mistakes(bt):
    """A loop vmcnt wait loosened past the DMA it covers, or the loop's lgkmcnt waits
    dropped, must both be reported."""
    prog = G.program("bf16", "f32", bt)
    top = prog.index("L_top_%=:")
    i = next(k for k in range(top, len(prog)) if prog[k].startswith("s_waitcnt vmcnt"))
    loose = prog[:i] + ["s_waitcnt vmcnt(40)"] + prog[i + 1:]
    assert Walk(loose, 16, bt).run().problems
    no_lgkm = [l for k, l in enumerate(prog) if not (k > top and l.startswith("s_waitcnt lgkmcnt"))]
    assert Walk(no_lgkm, 16, bt).run().problems
