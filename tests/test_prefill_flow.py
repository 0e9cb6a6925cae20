"""Control flow of the generated prefill main loop, checked on the CPU.

kernels/gen_prefill.py emits the loop as one asm statement.  Every wave of a
workgroup must pass the same number of s_barrier instructions (one per two K/V
periods), and before each barrier a wave must have waited for its own DMA share of
the K/V blocks the next two periods read.  Waves leave the compute loop at different blocks (the causal
diagonal), so this walks the scalar instructions of the program for every wave of
a range of (seq_len, start_pos, query block) shapes and checks both properties.
Vector instructions are skipped; vector compares that write scalar masks (the
rescale and residual-split decisions) take random values.
"""
import random
import re
import sys
from pathlib import Path

import pytest

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "tile-rs_amd" / "csrc" / "kernels"))
import gen_prefill as G  # noqa: E402

BQ, BKV = 256, 64


def operands(seq_len, start_pos, qb, wave):
    """The scalar operands prefill_asm.hpp hands to the asm statement (kernels/prefill_asm.hpp)."""
    q0 = qb * BQ
    q_hi = min(q0 + BQ, seq_len)
    nb = (start_pos + q_hi + BKV - 1) // BKV
    return {"nb": nb, "jd": (start_pos + q0 + 32 * wave + 1) // BKV,
            "jl": (start_pos + q0 + 32 * wave + 31) // BKV, "lds": 0, "wave2k": 2048 * wave,
            "kbase": 1 << 32, "vbase": 1 << 33, "kvlast": start_pos + seq_len - 1, "ok": (1 << 64) - 1}


def sreg(tok):
    if tok == "m0":
        return tok, False
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", tok)
    if m:
        return f"s{m.group(1)}", True
    m = re.fullmatch(r"s(\d+)", tok)
    return (tok, False) if m else (None, False)


class Wave:
    def __init__(self, prog, ops, rng):
        self.prog = [l.strip() for l in prog]
        self.labels = {l[:-1]: i for i, l in enumerate(self.prog) if l.endswith(":")}
        self.ops = {G.OP[k]: v for k, v in ops.items() if k in G.OP}
        self.s = {}
        self.exec = (1 << 64) - 1
        self.scc = 0
        self.rng = rng
        self.vmem = []            # kv0 of each vector memory op in issue order (None: not a DMA)
        self.barriers = []        # (s58, completed DMA kv0 set) at each barrier
        self.done_upto = 0        # vmem ops known complete (prefix length)
        self.mfmas = 0
        self.kv = {}              # block (kv0) each DMA address register was computed for

    def val(self, tok):
        tok = tok.strip()
        if tok == "exec":
            return self.exec
        if tok.startswith("%"):
            return self.ops[int(tok[1:])]
        r, _ = sreg(tok)
        if r is not None:
            return self.s.get(r, 0)
        return int(tok, 0)

    def put(self, tok, v):
        if tok == "exec":
            self.exec = v
        else:
            r, _ = sreg(tok)
            assert r is not None, tok
            self.s[r] = v

    def run(self, limit=2_000_000):
        pc, steps = 0, 0
        while pc < len(self.prog):
            steps += 1
            assert steps < limit, "no exit"
            line = self.prog[pc]
            pc += 1
            if not line or line.endswith(":"):
                continue
            op, _, rest = line.partition(" ")
            a = [x.strip() for x in rest.split(",")] if rest else []
            if op.startswith("global_load") or op.startswith("global_store"):
                real_dma = op == "global_load_lds_dwordx4" and self.exec != 0
                self.vmem.append(self.kv[a[0]] if real_dma else None)
            elif op in ("v_add_u32", "v_add3_u32") and a[0] in ("v16", "v17", "v18") and a[1].startswith("s"):
                # a DMA address: row = block kv0 (an SGPR) + lane offsets
                self.kv[a[0]] = self.val(a[1])
            elif op.startswith("v_mfma"):
                self.mfmas += 1
            elif op.startswith("v_cmp") and a and a[0].startswith("s["):
                self.put(a[0], self.rng.choice([0, 1, 1 << 40]))
            elif op.startswith("v_") or op.startswith("ds_") or op in ("s_nop",):
                pass
            elif op == "s_waitcnt":
                m = re.search(r"vmcnt\((\d+)\)", rest)
                if m:
                    self.done_upto = max(self.done_upto, len(self.vmem) - int(m.group(1)))
            elif op == "s_barrier":
                done = {kv for kv in self.vmem[:self.done_upto] if kv is not None}
                self.barriers.append((self.s.get("s58", -1), done))
            elif op in ("s_mov_b32", "s_mov_b64"):
                self.put(a[0], self.val(a[1]))
            elif op in ("s_add_u32", "s_addc_u32"):
                self.put(a[0], (self.val(a[1]) + self.val(a[2])) & 0xffffffff)
            elif op == "s_sub_u32":
                self.put(a[0], (self.val(a[1]) - self.val(a[2])) & 0xffffffff)
            elif op == "s_min_u32":
                self.put(a[0], min(self.val(a[1]), self.val(a[2])))
            elif op == "s_max_i32":
                sv = lambda x: x - (1 << 32) if x & (1 << 31) else x
                self.put(a[0], max(sv(self.val(a[1])), sv(self.val(a[2]))) & 0xffffffff)
            elif op == "s_or_b64":
                self.put(a[0], self.val(a[1]) | self.val(a[2]))
            elif op == "s_cselect_b32":
                self.put(a[0], self.val(a[1]) if self.scc else self.val(a[2]))
            elif op.startswith("s_cmp_"):
                x, y = self.val(a[0]), self.val(a[1])
                self.scc = int({"ge": x >= y, "gt": x > y, "lt": x < y, "eq": x == y,
                                "lg": x != y}[op.split("_")[2]])
            elif op in ("s_cbranch_scc0", "s_cbranch_scc1", "s_branch"):
                if op == "s_branch" or self.scc == int(op[-1]):
                    pc = self.labels[a[0]]
            else:
                raise AssertionError("unmodelled scalar instruction: " + line)
        return self


PROG = G.Gen("bf16").program()
PROGS = {128: PROG, 64: G.Gen("bf16", False, 64).program()}

SHAPES = [(1, 0), (40, 0), (64, 0), (65, 0), (200, 0), (256, 0), (300, 0), (700, 0),
          (1000, 0), (130, 5), (256, 64), (100, 1000), (513, 77)]


@pytest.mark.parametrize("head_dim", [128, 64])
@pytest.mark.parametrize("seq_len,start_pos", SHAPES)
def test_every_wave_passes_the_same_barriers(seq_len, start_pos, head_dim):
    rng = random.Random(seq_len * 131 + start_pos)
    for qb in range((seq_len + BQ - 1) // BQ):
        counts = set()
        for wave in range(8):
            ops = operands(seq_len, start_pos, qb, wave)
            w = Wave(PROGS[head_dim], ops, rng).run()
            nb = ops["nb"]
            counts.add(len(w.barriers))
            # one barrier after the prologue, then one per even period j = 0 .. nb-2
            want = 1 + (len(range(0, nb - 1, 2)) if nb >= 2 else 0)
            assert len(w.barriers) == want, (seq_len, start_pos, qb, wave, len(w.barriers), want)
            # before the barrier of even period j this wave's DMA of blocks j+1 and j+2
            # (all that periods j and j+1 read) has been issued and has landed; the
            # prologue's barrier covers block 0
            issued = {kv for kv in w.vmem if kv is not None}
            for i, (j, done) in enumerate(w.barriers):
                assert i == 0 or j % 2 == 0, (seq_len, start_pos, qb, wave, i, j)
                for need in ([0] if i == 0 else [BKV * (j + 1), BKV * (j + 2)]):
                    if need < BKV * nb:
                        assert need in issued and need in done, (seq_len, start_pos, qb, wave, i, j, need)
            # every DMA of the ring was issued (blocks 0 .. nb-1, one real batch each)
            assert {kv for kv in w.vmem if kv is not None} >= set(range(0, BKV * nb, BKV))
        assert len(counts) == 1


def test_walk_finds_a_missing_wait():
    """Planted mistake: without the vmcnt(0) waits of the even loop tops, blocks j+1
    and j+2 are not known to have landed at the barrier of period j."""
    prog = [l for l in PROG if l.strip() != "s_waitcnt vmcnt(0)"]
    ops = operands(1000, 0, 3, 7)
    w = Wave(prog, ops, random.Random(3)).run()
    missing = [(j, need) for i, (j, done) in enumerate(w.barriers) if i > 0
               for need in (BKV * (j + 1), BKV * (j + 2)) if need < BKV * ops["nb"] and need not in done]
    assert missing


@pytest.mark.parametrize("head_dim", [128, 64])
def test_waves_past_the_diagonal_drain(head_dim):
    """A wave whose rows end before the workgroup's last block skips the compute of the
    fully masked periods (wave 0 of a 256-row block: 3 of its 4 diagonal periods)."""
    ops = operands(256, 0, 0, 0)
    assert ops["jl"] == 0 and ops["nb"] == 4
    w0 = Wave(PROGS[head_dim], ops, random.Random(1)).run()
    w7 = Wave(PROGS[head_dim], operands(256, 0, 0, 7), random.Random(1)).run()
    assert len(w0.barriers) == len(w7.barriers) == 3
    # MFMAs per block: n QK and n PV (n = 16 at head_dim 128, 8 at 64); wave 0: S(0),
    # the PV of its only block and at most 4 residual steps of n/4; wave 7: S(0), three
    # periods and the last PV block
    n = head_dim // 8
    assert w0.mfmas <= n + n + n
    assert w7.mfmas >= n + 3 * 2 * n + n


# ---------------------------------------------------------------------------
# Issue hazards of the hand-written loop.  The assembler inserts no wait states
# into an asm statement, so the generator must: on gfx950 a non-transcendental
# VALU instruction that reads or writes the destination of a transcendental op
# (v_exp/v_rcp/v_log/v_sqrt/v_rsq) in the very next issue slot can see the value
# from before it (found as run-to-run output drift of 1-2 bf16 ulp at config 4).
# ---------------------------------------------------------------------------
TRANS = ("v_exp_f32", "v_rcp_f32", "v_log_f32", "v_sqrt_f32", "v_rsq_f32")


def vregs(text):
    out = set()
    for a, b in re.findall(r"\bv\[(\d+):(\d+)\]", text):
        out |= set(range(int(a), int(b) + 1))
    out |= {int(a) for a in re.findall(r"\bv(\d+)\b", text)}
    return out


def trans_hazards(prog):
    """(trans line, next line) pairs where the instruction issued right after a
    transcendental op touches its destination with no wait state between.  Labels
    are transparent; an unconditional branch continues at its target."""
    lines = [l.strip() for l in prog]
    labels = {l[:-1]: i for i, l in enumerate(lines) if l.endswith(":")}

    def next_issued(i):
        seen = set()
        while i < len(lines) and i not in seen:
            seen.add(i)
            ln = lines[i]
            if ln.endswith(":"):
                i += 1
            elif ln.startswith("s_branch "):
                i = labels[ln.split()[1]] + 1
            else:
                return ln
        return None

    bad = []
    for i, ln in enumerate(lines):
        op = ln.split()[0] if ln else ""
        if op not in TRANS:
            continue
        dst = vregs(ln.split(None, 1)[1].split(",")[0])
        nxt = next_issued(i + 1)
        if nxt is None or not nxt.startswith("v_") or nxt.split()[0] in TRANS:
            continue
        if dst & vregs(nxt.split(None, 1)[1]):
            bad.append((ln, nxt))
    return bad


def test_trans_hazard_check_finds_a_planted_case():
    planted = ["v_exp_f32 v248, v248", "Lx_%=:", "v_mul_f32 v248, %17, v248"]
    assert trans_hazards(planted) == [("v_exp_f32 v248, v248", "v_mul_f32 v248, %17, v248")]
    assert trans_hazards(["v_exp_f32 v40, v40", "s_branch L1", "L1:", "v_add_f32 v41, v41, v40"])
    assert not trans_hazards(["v_exp_f32 v40, v40", "s_nop 0", "v_add_f32 v41, v41, v40"])
    assert not trans_hazards(["v_exp_f32 v40, v40", "v_exp_f32 v42, v42", "v_add_f32 v41, v41, v40"])


@pytest.mark.parametrize("head_dim", [128, 64])
@pytest.mark.parametrize("partial", [False, True])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_no_trans_forwarding_hazard(dt, partial, head_dim):
    assert trans_hazards(G.Gen(dt, partial, head_dim).program()) == []


@pytest.mark.parametrize("head_dim", [128, 64])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_split_part_program_differs_only_in_the_epilogue(dt, head_dim):
    """The split-KV part program runs the same loop; only the code after the loop
    (f32 partial rows instead of normalized 16-bit O) differs."""
    full, part = G.Gen(dt, False, head_dim).program(), G.Gen(dt, True, head_dim).program()
    cut = next(i for i, l in enumerate(full) if l.startswith("v_rcp_f32"))
    assert part[:cut] == full[:cut]
    assert not any(l.startswith("v_rcp_f32") for l in part)
    stores = [l for l in part if l.startswith("global_store")]
    assert len(stores) == head_dim // 8 + 1 and stores[-1].endswith(f"offset:{4 * head_dim}")


# ---------------------------------------------------------------------------
# Static checks of the program text: the asm statement gets no checking from the
# compiler beyond assembling each line, so a branch to a label outside the
# program, a register the statement does not own, or an accumulation register
# (AGPR: the unified register file then has to hold 256 VGPRs plus the AGPRs,
# more than a 512-thread workgroup may use) would only show on the GPU.
# ---------------------------------------------------------------------------
BRANCHES = ("s_branch", "s_cbranch_scc0", "s_cbranch_scc1", "s_cbranch_vccz", "s_cbranch_vccnz",
            "s_cbranch_execz", "s_cbranch_execnz")
CLOBBER_V = set(range(16, 256))
CLOBBER_S = set(range(48, 96))


def sregs(text):
    out = set()
    for a, b in re.findall(r"\bs\[(\d+):(\d+)\]", text):
        out |= set(range(int(a), int(b) + 1))
    out |= {int(a) for a in re.findall(r"\bs(\d+)\b", text)}
    return out


def static_problems(prog):
    lines = [l.strip() for l in prog]
    defs = [l[:-1] for l in lines if l.endswith(":")]
    bad = [f"label defined twice: {d}" for d in set(defs) if defs.count(d) > 1]
    labels = set(defs)
    for ln in lines:
        op = ln.split()[0] if ln else ""
        if op.startswith("s_branch") or op.startswith("s_cbranch") or op.startswith("s_setpc") \
                or op.startswith("s_swappc"):
            if op not in BRANCHES:
                bad.append("unexpected control transfer: " + ln)
            elif ln.split()[1] not in labels:
                bad.append("branch outside the program: " + ln)
        if ln.endswith(":") or not op:
            continue
        body = ln.split(None, 1)[1] if " " in ln else ""
        if re.search(r"\ba\[\d+:\d+\]|\ba\d+\b|accvgpr", ln):
            bad.append("AGPR operand: " + ln)
        if vregs(body) - CLOBBER_V:
            bad.append("VGPR outside the clobber list: " + ln)
        if sregs(body) - CLOBBER_S:
            bad.append("SGPR outside the clobber list: " + ln)
        for a, b in re.findall(r"\bv\[(\d+):(\d+)\]", body):
            if int(a) % 2:
                bad.append("odd-aligned VGPR tuple: " + ln)
    return bad


def test_static_check_finds_planted_cases():
    assert static_problems(["s_branch L9_0"])
    assert static_problems(["L1:", "L1:"])
    assert static_problems(["v_accvgpr_write_b32 a3, v40"])
    assert static_problems(["v_mfma_f32_32x32x16_bf16 a[0:15], v[40:43], v[44:47], a[0:15]"])
    assert static_problems(["v_mov_b32 v3, v40"])
    assert static_problems(["s_mov_b32 s20, s48"])
    assert static_problems(["ds_read_b64 v[41:42], v40"])
    assert static_problems(["s_setpc_b64 s[48:49]"])
    assert not static_problems(["L1:", "s_cbranch_scc1 L1", "v_mov_b32 v40, %3"])


@pytest.mark.parametrize("head_dim", [128, 64])
@pytest.mark.parametrize("partial", [False, True])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_program_text_is_self_contained(dt, partial, head_dim):
    prog = G.Gen(dt, partial, head_dim).program()
    assert static_problems(prog) == []
    # m0 is saved on entry and restored as the last instruction (single exit)
    assert prog[0] == "s_mov_b32 s52, m0" and prog[-1] == "s_mov_b32 m0, s52"
    assert not any("s52" in l for l in prog[1:-1])


def test_clobber_list_matches_the_checked_sets():
    text = Path(G.__file__).read_text()
    assert 'for k in range(16, 256)' in text and 'for k in range(48, 96)' in text


# ---------------------------------------------------------------------------
# K stage layout: the DMA lanes' (row, chunk) targets and the fragment reads must
# agree.  The lane operands klane, krow and kcol are restated from
# kernels/prefill_asm.hpp; the read registers, their XORs and the immediates are
# taken from the generated program.
# ---------------------------------------------------------------------------
def k_layout(head_dim, klane, krow, kcol, prog):
    rb = 2 * head_dim
    lds = {}
    for w in range(8):
        for j in range(head_dim // 64):
            for lane in range(64):
                addr = (2048 if head_dim == 128 else 1024) * w + 1024 * j + 16 * lane
                assert kcol(w, lane) + 16 <= rb
                assert addr not in lds
                lds[addr] = (krow(w, lane) + 8 * j, kcol(w, lane) // 16)
    assert sorted(lds.values()) == [(r, c) for r in range(64) for c in range(head_dim // 8)]
    # the period's K fragment reads in issue order, and each base register's XOR
    xor = {G.KADDR: 0}
    for ln in prog:
        m = re.fullmatch(r"v_xor_b32 (v\d+), (\d+), " + G.KADDR, ln.strip())
        if m:
            xor[m.group(1)] = int(m.group(2))
    reads = [re.fullmatch(r"ds_read_b128 v\[\d+:\d+\], (v\d+) offset:(\d+)", ln.strip()) for ln in prog]
    reads = [(m.group(1), int(m.group(2))) for m in reads if m and m.group(1) in xor]
    nds = head_dim // 16
    frags = reads[:2 * nds]            # S(0) in the prologue: (ds, kt) in issue order
    bad = []
    for i, (reg, off) in enumerate(frags):
        ds, kt = i // 2, i % 2
        for lane in range(64):
            a = (klane(lane) ^ xor[reg]) + off
            want = (32 * kt + (lane & 31), 2 * ds + (lane >> 5))
            if lds.get(a) != want:
                bad.append((ds, kt, lane, lds.get(a), want))
        # a ds_read_b128 conflict window: lanes l .. l+7 with l+16 .. l+23 (measured:
        # the GEMM's A layout, c ^ (r & 7) over 16 rows, has no conflicts; this K layout
        # with c ^ (r & 7) over 32 rows had 32% of LDS-active cycles in conflicts)
        for base in (0, 8, 32, 40):
            lanes = list(range(base, base + 8)) + list(range(base + 16, base + 24))
            pos = [((klane(l) ^ xor[reg]) + off) % 256 // 16 for l in lanes]
            if len(set(pos)) != len(pos):
                bad.append(("conflict", ds, kt, base))
    return bad


def kswz(r):
    return ((r >> 1) & 3) | ((r >> 2) & 4)


def klane_hpp(lane):
    l32, g = lane & 31, lane >> 5
    return 128 * l32 + 16 * (g ^ kswz(l32))


@pytest.mark.parametrize("head_dim", [128, 64])
def test_k_stage_layout(head_dim):
    krow = lambda w, lane: (16 * (w & 3) if head_dim == 128 else 8 * w) + (lane >> 3)
    kcol = lambda w, lane: (128 * (w >> 2) if head_dim == 128 else 0) + 16 * ((lane & 7) ^ kswz(krow(w, lane)))
    assert k_layout(head_dim, klane_hpp, krow, kcol, PROGS[head_dim]) == []


def test_k_stage_layout_check_finds_a_planted_mistake():
    """The unswizzled chunk order on the DMA side: reads land on the wrong chunks."""
    krow = lambda w, lane: 16 * (w & 3) + (lane >> 3)
    kcol = lambda w, lane: 128 * (w >> 2) + 16 * (lane & 7)
    assert k_layout(128, klane_hpp, krow, kcol, PROGS[128])


def test_k_stage_conflict_check_finds_the_rows_16_apart():
    """Swizzle r & 7: the reads find the right data but rows r and r + 16 share banks in
    one conflict window."""
    krow = lambda w, lane: 16 * (w & 3) + (lane >> 3)
    kcol = lambda w, lane: 128 * (w >> 2) + 16 * ((lane & 7) ^ (krow(w, lane) & 7))
    klane = lambda lane: 128 * (lane & 31) + 16 * ((lane >> 5) ^ (lane & 7))
    bad = k_layout(128, klane, krow, kcol, PROGS[128])
    assert bad and all(b[0] == "conflict" for b in bad)
