"""Generate the main loop of the causal GQA prefill kernel (head_dim 128, bf16/f16)
as gfx950 assembly for one inline-asm statement (prefill_asm.hpp wraps it).

Semantics are those of the reference's fused prefill (causal softmax(Q.K^T *
rsqrt(D)) . V over positions <= start_pos + query row;
/root/reference/crates/rustc_codegen_tile/src/mlir_to_msl.rs:10928-11009), computed
as a flash-attention online softmax in base 2 with lazy rescaling.

Workgroup = 8 waves = 256 query rows of one (batch, head); wave w owns rows
[32w, 32w+32) and runs two per SIMD.  KV advances 64 positions at a time through
a ring of NS LDS stages filled by global_load_lds_dwordx4 (no register staging):
  K stage [2 halves][64 rows][8 chunks] x 16 B (head_dim 64: one half), chunk c of
           row r at c ^ f(r), f(r) = bits 1-2 and 4 of r (prefill_asm.hpp): one DMA
           instruction writes 8 rows x 128 bytes, so every K fetch is a whole cache
           line (4 us faster at config 4 than 16 rows x 64 bytes, same bits); a
           fragment read is one of four lane bases (XOR 32 q, q = ds & 3) plus an
           immediate, without bank conflicts (another 2-5 us);
  V stage [64 kv][128 d] row-major with chunk c of row r at c ^ 4(r & 3), read as
           V^T with ds_read_b64_tr_b16.
Per wave and period j (S = scores of 64 kv x 32 queries, as S^T accumulators):
    MFMA:  S(j+1) = K(j+1).Q^T (16 x v_mfma_f32_32x32x16), then
           O^T += V(j)^T.P(j)^T (16 MFMAs), fragments prefetched PD ahead
    VALU:  phase B of block j (rescale check, 16-bit P, second half of the
           exponentials, row sum, split decision), then phase A of block j+1
           (causal mask, row max, running max, first half of the exponentials)
           once S(j+1) is complete; both spread between the MFMAs.
A 16-position PV step whose largest probability exceeds 1/ratio of the row's
running sum also gets its 16-bit residual P - hi(P) multiplied in (out of line,
only for those steps: 4 MFMAs per step instead of 16 per block).  Scores
are double-buffered by block parity, so the loop is unrolled by two.  One
s_barrier per two periods, at even j: before it each wave waits for its DMA share
of blocks j+1 and j+2 (all it reads until the next barrier); after it every wave
has finished period j-1, so the stages of blocks j-2 and j-1 are free, and period j
refills the first with block j+3, period j+1 the second with block j+4 (one DMA
block per period, each issued one or two periods before the barrier that publishes
it).  Measured at config 4 against one barrier per period: 10-17 us faster, same
bits; issuing both blocks in the even period was not faster.
A wave whose rows end before the workgroup's last block (the causal diagonal:
wave 0 of a 256-row block needs one of the last four blocks) leaves the compute
loop after its last unmasked block jl (whose period runs PV(jl) without the
all-masked S(jl+1)) and drains: each remaining period only does the period's
waits, barrier and DMA issue, so every wave passes the same barriers (tests/test_prefill_flow.py walks the scalar
control flow of this program for every wave and checks it).

Register map (VGPRs only; the asm statement clobbers v16-v255, s48-s95):
  v16 v17 v18 DMA offsets, v19 v20 temps, v21-v23 K fragment bases 1-3,
  v[24:27] v[28:31] per-step score maxima
  (by block parity),
  v[32:63] S (even blocks), v[64:95] S (odd blocks), v[96:111] P,
  v[112:143] fragment ring (8 x 4), v[144:207] O^T (4 d-tiles x 16),
  v[208:239] Q^T fragments (8 x 4),
  v240-247 m l lim mblk mnew alpha ls0 ls1, v248 v249 temps, v250 -inf,
  v251 K address, v252-255 V^T addresses.
SGPRs: s[48:49] K base, s[56:57] V base, s58 j, s59 nb-1 (jl and jd are
  operands), s60 stage of
  block j+1, s61 stage of block j, s62 s63 DMA stage and kv0 of an even period,
  s53 s54 those of the odd period after it, s64 s68 temps,
  s65 stage end, s[66:67] saved exec, s[70:71] grow mask, s[74:75] s[92:93] DMA exec
  (even, odd period),
  s[76:77] full exec, s[78:79] split mask (any step), s[80:81] mask compare,
  s[84:91] split masks of the four PV steps.

Usage: python gen_prefill.py <out.inc>   (run by the library build)
"""
import sys
from pathlib import Path

NS = 5          # LDS ring stages of 64 KV positions (K 16 KB + V 16 KB each)
PD = 6          # fragment prefetch distance (fragments in flight ahead of their MFMA)
RING = 8        # fragment ring size (4 VGPRs per fragment)

# operand numbers of the asm statement (see prefill_asm.hpp)
OP = dict(qp=0, op=1, lim=2, klane=3, vlane=4, krow=5, kcol=6, vrow=7, vcol=8,
          kbase=9, vbase=10, kvlast=11, nb=12, jd=13, lds=14, wave2k=15,
          scale=16, lratio=17, ok=18, jl=19)


def o(name):
    return f"%{OP[name]}"


S_BASE = [32, 64]
P_BASE = 96
RING_BASE = 112
O_BASE = 144
Q_BASE = 208
STB = 240
X0, X1, NINF, KADDR = "v248", "v249", "v250", "v251"
# K fragment bases: lane base XOR 32 q for q = ds & 3 (chunk 2 ds + g is stored at
# (2 ds + g) ^ f(row), so ds & 3 enters as an XOR of chunk bits 1-2)
KADDRS = [KADDR, "v21", "v22", "v23"]
# Raw score maxima of the block's four 16-position PV steps (this lane's 8 scores of
# each), by block parity: the residual split is decided, and run, per step.
STEPMAX = [24, 28]
SPLIT_MASK = ["s[84:85]", "s[86:87]", "s[88:89]", "s[90:91]"]
VADDR = [252, 253, 254, 255]
DK, DV = "v16", ["v17", "v18"]
TA, TB = "v19", "v20"


def st(name):
    return f"v{STB + ['m', 'l', 'lim', 'mblk', 'mnew', 'alpha', 'ls0', 'ls1'].index(name)}"


def names(dt):
    mn = "v_mfma_f32_32x32x16_bf16" if dt == "bf16" else "v_mfma_f32_32x32x16_f16"
    cvt = "v_cvt_pk_bf16_f32" if dt == "bf16" else "v_cvt_pk_f16_f32"
    return mn, cvt


def vr(a, b):
    return f"v[{a}:{b}]"


INF = 10 ** 9


class Gen:
    def __init__(self, dt, partial=False, d=128):
        assert d in (128, 64)
        self.dt = dt
        self.partial = partial
        self.D = d
        self.NDS = d // 16          # 16-deep QK MFMA steps along the head dim
        self.NDT = d // 32          # 32-wide O^T tiles (PV MFMAs per 16-position step)
        self.RB = 2 * d             # bytes of a K or V row
        self.KRG = 16 * self.RB     # bytes of a K row group (16 rows, all chunks)
        self.KB = 64 * self.RB      # bytes of the K (or V) half of a stage
        self.SS = 2 * self.KB       # bytes of a ring stage
        self.NLDK = d // 64         # K (and V) DMA loads per wave and block
        self.NLD = 2 * self.NLDK
        self.SHIFT = 8 if d == 128 else 7
        self.mn, self.cvt = names(dt)
        self.uid = 0
        self.ool = []

    def label(self, base):
        self.uid += 1
        return f"L{base}{self.uid}_%="

    # ---------------- fragment streams ----------------
    def qk_frags(self, par):
        out = []
        for i in range(2 * self.NDS):
            ds, kt = i // 2, i % 2
            d0 = S_BASE[par] + 16 * kt
            q0 = Q_BASE + 4 * ds
            src_c = "0" if ds == 0 else vr(d0, d0 + 15)
            out.append(dict(
                reads=lambda R, kt=kt, ds=ds: [f"ds_read_b128 {vr(R, R + 3)}, {KADDRS[ds & 3]} offset:{8192 * (ds >> 2) + 4096 * kt}"],
                mfma=lambda R, d0=d0, q0=q0, src_c=src_c:
                    f"{self.mn} {vr(d0, d0 + 15)}, {vr(R, R + 3)}, {vr(q0, q0 + 3)}, {src_c}",
                pdep=None))
        return out

    def pv_frags(self):
        out = []
        for k in range(4 * self.NDT):
            stp, dtl = k // self.NDT, k % self.NDT
            ob = O_BASE + 16 * dtl
            pb = P_BASE + 4 * stp
            va = f"v{VADDR[dtl]}"
            out.append(dict(
                reads=lambda R, va=va, stp=stp: [f"ds_read_b64_tr_b16 {vr(R, R + 1)}, {va} offset:{16 * self.RB * stp}",
                                                 f"ds_read_b64_tr_b16 {vr(R + 2, R + 3)}, {va} offset:{16 * self.RB * stp + 8 * self.RB}"],
                mfma=lambda R, ob=ob, pb=pb: f"{self.mn} {vr(ob, ob + 15)}, {vr(R, R + 3)}, {vr(pb, pb + 3)}, {vr(ob, ob + 15)}",
                pdep=stp))
        return out

    # ---------------- softmax ----------------
    def phase_a(self, par, masked, earliest):
        """Mask, row max, running max and alpha (grow mask -> s[70:71]),
        exponentials and row sums of scores 0..15."""
        S = [f"v{S_BASE[par] + e}" for e in range(32)]
        scale = o("scale")
        m_run, m_blk, m_new, alpha = st("m"), st("mblk"), st("mnew"), st("alpha")
        ls0, ls1 = st("ls0"), st("ls1")
        L = []
        if masked:
            for e in range(32):
                kt, r = e // 16, e % 16
                c = 32 * kt + 8 * (r >> 2) + (r & 3)
                L.append([f"v_cmp_lt_i32 s[80:81], {st('lim')}, {c}", f"v_cndmask_b32 {S[e]}, {S[e]}, {NINF}, s[80:81]"])
        # per-step maxima (PV step t holds this lane's scores 8t .. 8t+7), four chains
        mx = [f"v{STEPMAX[par] + t}" for t in range(4)]
        seqs = []
        for t in range(4):
            g = list(range(8 * t, 8 * t + 8))
            seqs.append([f"v_max3_f32 {mx[t]}, {S[g[0]]}, {S[g[1]]}, {S[g[2]]}",
                         f"v_max3_f32 {mx[t]}, {mx[t]}, {S[g[3]]}, {S[g[4]]}",
                         f"v_max3_f32 {mx[t]}, {mx[t]}, {S[g[5]]}, {S[g[6]]}",
                         f"v_max_f32 {mx[t]}, {mx[t]}, {S[g[7]]}"])
        for i in range(4):
            for q in seqs:
                L.append([q[i]])
        L.append([f"v_max3_f32 {X0}, {mx[0]}, {mx[1]}, {mx[2]}"])
        L.append([f"v_max_f32 {X0}, {X0}, {mx[3]}"])
        L.append([f"v_mov_b32 {X1}, {X0}", "s_nop 1", f"v_permlane32_swap_b32 {X0}, {X1}", "s_nop 1"])
        L.append([f"v_max_f32 {X0}, {X0}, {X1}"])
        L.append([f"v_mul_f32 {m_blk}, {scale}, {X0}"])
        L.append([f"v_add_f32 {X1}, 0x41000000, {m_run}"])
        L.append([f"v_max_f32 {X0}, {m_run}, {m_blk}"])
        L.append([f"v_cmp_gt_f32 s[70:71], {m_blk}, {X1}"])
        L.append([f"v_cndmask_b32 {m_new}, {m_run}, {X0}, s[70:71]"])
        L.append([f"v_sub_f32 {X1}, {m_run}, {m_new}"])
        L.append([f"v_exp_f32 {alpha}, {X1}"])
        L.append([f"v_mov_b32 {m_run}, {m_new}"])
        L.append([f"v_mov_b32 {ls0}, 0", f"v_mov_b32 {ls1}, 0"])
        for g0 in range(0, 16, 4):
            for e in range(g0, g0 + 4):
                L.append([f"v_fma_f32 {S[e]}, {S[e]}, {scale}, -{m_new}"])
            for e in range(g0, g0 + 4):
                L.append([f"v_exp_f32 {S[e]}, {S[e]}"])
            for e in range(g0, g0 + 4):
                L.append([f"v_add_f32 {ls0 if e % 2 == 0 else ls1}, {ls0 if e % 2 == 0 else ls1}, {S[e]}"])
        return [dict(lines=x, deadline=INF, earliest=earliest) for x in L]

    def phase_b(self, par, pv0):
        """Rescale check (before the first PV MFMA at slot pv0), P st 0-1, the
        other 16 exponentials with P st 2-3, l update and split decision."""
        S = [f"v{S_BASE[par] + e}" for e in range(32)]
        P = [f"v{P_BASE + q}" for q in range(16)]
        scale, lratio = o("scale"), o("lratio")
        m_blk, m_new, alpha, l_run = st("mblk"), st("mnew"), st("alpha"), st("l")
        ls0, ls1 = st("ls0"), st("ls1")
        ops = []

        def add(lines, deadline=INF):
            ops.append(dict(lines=lines, deadline=deadline, earliest=-1))

        def pdl(q):
            return (pv0 + self.NDT * (q // 4) - 2) if q % 4 == 3 else INF
        lg, lb = self.label("grow"), self.label("growb")
        body = ["s_nop 7", "s_nop 7", "s_nop 7"]
        for k in range(16 * self.NDT):
            body.append(f"v_mul_f32 v{O_BASE + k}, {alpha}, v{O_BASE + k}")
        self.ool.append([f"{lg}:"] + body + [f"s_branch {lb}"])
        add(["s_cmp_lg_u64 s[70:71], 0", f"s_cbranch_scc1 {lg}", f"{lb}:"], pv0 - 1)
        for q in range(8):
            add([f"{self.cvt} {P[q]}, {S[2 * q]}, {S[2 * q + 1]}"], pdl(q))
        for g0 in range(16, 32, 4):
            for e in range(g0, g0 + 4):
                add([f"v_fma_f32 {S[e]}, {S[e]}, {scale}, -{m_new}"])
            for e in range(g0, g0 + 4):
                add([f"v_exp_f32 {S[e]}, {S[e]}"])
            for e in range(g0, g0 + 4):
                add([f"v_add_f32 {ls0 if e % 2 == 0 else ls1}, {ls0 if e % 2 == 0 else ls1}, {S[e]}"])
            for q in (g0 // 2, g0 // 2 + 1):
                add([f"{self.cvt} {P[q]}, {S[2 * q]}, {S[2 * q + 1]}"], pdl(q))
        add([f"v_add_f32 {X0}, {ls0}, {ls1}"])
        add([f"v_fma_f32 {l_run}, {l_run}, {alpha}, {X0}"])
        add([f"v_mov_b32 {X1}, {l_run}", f"v_mov_b32 {TA}, {l_run}", "s_nop 1",
             f"v_permlane32_swap_b32 {X1}, {TA}", "s_nop 1"])
        add([f"v_add_f32 {X1}, {X1}, {TA}"])
        # Split step t when its largest probability exceeds 1/ratio of the row's sum:
        # only those steps' residual MFMAs run (out of line, after the period).
        # Compared in the log2 domain: scale*mx - m_new + log2(ratio) > log2(sum), one
        # v_log per block instead of four v_exp.  The log's result is read four slots
        # later: a non-transcendental VALU op must not touch a transcendental op's
        # destination in the next issue slot (gfx950 trans forwarding).
        mx = [f"v{STEPMAX[par] + t}" for t in range(4)]
        add([f"v_log_f32 {X1}, {X1}"])
        add([f"v_subrev_f32 {X0}, {lratio}, {m_new}"])
        for t in range(4):
            add([f"v_fma_f32 {mx[t]}, {mx[t]}, {scale}, -{X0}"])
        for t in range(4):
            add([f"v_cmp_gt_f32 {SPLIT_MASK[t]}, {mx[t]}, {X1}"])
        add([f"s_or_b64 s[78:79], {SPLIT_MASK[0]}, {SPLIT_MASK[1]}",
             f"s_or_b64 s[78:79], s[78:79], {SPLIT_MASK[2]}",
             f"s_or_b64 s[78:79], s[78:79], {SPLIT_MASK[3]}"])
        return ops

    def split_tail(self, par):
        """Residual PV of the block whose P was just consumed (rare): runs after
        the period's last MFMA; lo = P - hi(P) overwrites P, fragments use the ring."""
        ls, lsb = self.label("split"), self.label("splitb")
        self.ool.append([f"{ls}:"] + self.residual(par) + [f"s_branch {lsb}"])
        return ["s_cmp_lg_u64 s[78:79], 0", f"s_cbranch_scc1 {ls}", f"{lsb}:"]

    def residual(self, par):
        """lo = P - hi(P) for the split steps only, and O^T += V^T . lo for them: per
        step, its four V fragments are read while lo is computed."""
        S = [f"v{S_BASE[par] + e}" for e in range(32)]
        P = [f"v{P_BASE + q}" for q in range(16)]
        # the period's last MFMAs may still read P: 16 wait states before overwriting it
        out = ["s_waitcnt lgkmcnt(0)", "s_nop 7", "s_nop 7"]
        for t in range(4):
            skip = self.label("rskip")
            out += [f"s_cmp_lg_u64 {SPLIT_MASK[t]}, 0", f"s_cbranch_scc0 {skip}"]
            for dtl in range(self.NDT):
                R = RING_BASE + 4 * dtl
                va = f"v{VADDR[dtl]}"
                out += [f"ds_read_b64_tr_b16 {vr(R, R + 1)}, {va} offset:{16 * self.RB * t}",
                        f"ds_read_b64_tr_b16 {vr(R + 2, R + 3)}, {va} offset:{16 * self.RB * t + 8 * self.RB}"]
            for q in range(4 * t, 4 * t + 4):
                if self.dt == "bf16":
                    out += [f"v_lshlrev_b32 {TA}, 16, {P[q]}", f"v_and_b32 {TB}, 0xffff0000, {P[q]}"]
                else:
                    out += [f"v_cvt_f32_f16 {TA}, {P[q]}", f"v_lshrrev_b32 {TB}, 16, {P[q]}",
                            f"v_cvt_f32_f16 {TB}, {TB}"]
                out += [f"v_sub_f32 {TA}, {S[2 * q]}, {TA}", f"v_sub_f32 {TB}, {S[2 * q + 1]}, {TB}",
                        f"{self.cvt} {P[q]}, {TA}, {TB}"]
            out.append("s_nop 2")
            pb = P_BASE + 4 * t
            for dtl in range(self.NDT):
                R = RING_BASE + 4 * dtl
                ob = O_BASE + 16 * dtl
                out.append(f"s_waitcnt lgkmcnt({2 * (self.NDT - 1 - dtl)})")
                out.append(f"{self.mn} {vr(ob, ob + 15)}, {vr(R, R + 3)}, {vr(pb, pb + 3)}, {vr(ob, ob + 15)}")
            # the ring slots are refilled by the next split step: its reads wait for these MFMAs
            out += ["s_nop 7", "s_nop 7", f"{skip}:"]
        out += ["s_nop 7", "s_nop 7", "s_nop 3"]
        return out

    # ---------------- scheduler ----------------
    def schedule(self, frags, ops, pre_quota=12):
        n = len(frags)
        ring = [RING_BASE + 4 * (f % RING) for f in range(n)]
        reads = [fr["reads"](ring[f]) for f, fr in enumerate(frags)]
        tail = [op for op in ops if op["earliest"] >= n]
        ops = [op for op in ops if op["earliest"] < n]
        dl = [min(op["deadline"], n - 1) for op in ops]
        for i in range(len(ops) - 2, -1, -1):
            dl[i] = min(dl[i], dl[i + 1])
        out = []
        issued = min(PD - 1, n)
        for f in range(issued):
            out += reads[f]
        pos = 0
        p_slot = {}

        def emit_ops(slot, quota):
            nonlocal pos
            k = 0
            while pos < len(ops):
                op = ops[pos]
                forced = dl[pos] <= slot
                if not forced and (k >= quota or op["earliest"] > slot):
                    break
                if op["earliest"] > slot:
                    raise RuntimeError(f"infeasible op {op['lines']} at slot {slot}")
                out.extend(op["lines"])
                for ln in op["lines"]:
                    if ln.startswith(self.cvt):
                        reg = int(ln.split()[1].rstrip(",")[1:])
                        if P_BASE <= reg < P_BASE + 16:
                            p_slot[(reg - P_BASE) // 4] = slot
                pos += 1
                k += 1
        emit_ops(-1, pre_quota)
        for s in range(n):
            if issued < n:
                out += reads[issued]
                issued += 1
            later = sum(len(reads[x]) for x in range(s + 1, issued))
            out.append(f"s_waitcnt lgkmcnt({min(later, 15)})")
            pdep = frags[s]["pdep"]
            if pdep is not None and p_slot.get(pdep, -99) >= s - 1:
                out.append("s_nop 2")
            out.append(frags[s]["mfma"](ring[s]))
            rem_ops, rem_slots = len(ops) - pos, n - s
            emit_ops(s, -(-rem_ops // rem_slots))
        for op in ops[pos:]:
            out.extend(op["lines"])
        if tail:
            out += ["s_nop 7", "s_nop 7", "s_nop 3"]
            for op in tail:
                out.extend(op["lines"])
        return out

    # ---------------- DMA ----------------
    def dma_lines(self, masked_exec, st_="s62", kv="s63", ex="s[74:75]"):
        """Block kv into the stage at st_: two K and two V loads per lane."""
        ex0 = [f"s_mov_b64 exec, {ex}"] if masked_exec else []
        ex1 = ["s_mov_b64 exec, s[76:77]"] if masked_exec else []
        groups = [[f"v_add_u32 {DK}, {kv}, {o('krow')}", f"v_min_u32 {DK}, {o('kvlast')}, {DK}",
                   f"v_lshl_add_u32 {DK}, {DK}, {self.SHIFT}, {o('kcol')}", f"s_add_u32 s64, {st_}, {o('wave2k')}"]]
        # an LDS DMA reads m0 one wait state after it is written (the exec write, when
        # there is one, is that wait state)
        w0 = ex0 or ["s_nop 0"]
        for j in range(self.NLDK):
            if j:
                # K unit j holds 8 more rows at the same columns (the swizzle follows r & 7)
                groups.append([f"v_add3_u32 {DK}, {kv}, {o('krow')}, {8 * j}", f"v_min_u32 {DK}, {o('kvlast')}, {DK}",
                               f"v_lshl_add_u32 {DK}, {DK}, {self.SHIFT}, {o('kcol')}"])
            groups.append([f"s_add_u32 m0, s64, {1024 * j}"] + w0 +
                          [f"global_load_lds_dwordx4 {DK}, s[48:49]"] + ex1)
        for j in range(self.NLDK):
            groups.append([f"v_add3_u32 {DV[j]}, {kv}, {o('vrow')}, {4 * j}", f"v_min_u32 {DV[j]}, {o('kvlast')}, {DV[j]}",
                           f"v_lshl_add_u32 {DV[j]}, {DV[j]}, {self.SHIFT}, {o('vcol')}"])
            groups.append([f"s_add_u32 m0, s64, {self.KB + 1024 * j}"] + w0 +
                          [f"global_load_lds_dwordx4 {DV[j]}, s[56:57]"] + ex1)
        return groups

    def rotate(self, sreg):
        return [f"s_add_u32 {sreg}, {sreg}, {self.SS}", f"s_cmp_ge_u32 {sreg}, s65",
                f"s_cselect_b32 {sreg}, {o('lds')}, {sreg}"]

    def addr_k(self, sreg):
        out = [f"v_add_u32 {KADDR}, {sreg}, {o('klane')}"]
        for q in range(1, 4):
            out.append(f"v_xor_b32 {KADDRS[q]}, {32 * q}, {KADDR}")
        return out

    def addr_v(self, sreg):
        out = ["s_add_u32 s68, " + sreg + f", {self.KB}", f"v_add_u32 v{VADDR[0]}, s68, {o('vlane')}"]
        for d in range(1, self.NDT):
            out.append(f"v_xor_b32 v{VADDR[d]}, {d << 6}, v{VADDR[0]}")
        return out

    # ---------------- bodies ----------------
    def period(self, par, masked):
        frags = self.qk_frags(1 - par) + self.pv_frags()
        nqk = 2 * self.NDS
        # every period j issues block j+3: even ones from s62/s63 (exec s[74:75]), odd
        # ones from s53/s54 (exec s[92:93]); the even loop top sets both
        dma = self.dma_lines(True) if par == 0 else self.dma_lines(True, "s53", "s54", "s[92:93]")
        ops = [dict(lines=g, deadline=min(12, nqk - 2), earliest=-1) for g in dma]
        ops += self.phase_b(par, pv0=nqk) + self.phase_a(1 - par, masked, earliest=nqk + 2)
        pre = self.addr_k("s60") + self.addr_v("s61")
        body = self.schedule(frags, ops)
        tail = ["s_nop 7", "s_nop 7"] + self.split_tail(par)
        return pre + body + tail

    def last(self, par):
        frags = self.pv_frags()
        ops = self.phase_b(par, pv0=0)
        pre = self.addr_v("s61")
        return pre + self.schedule(frags, ops, pre_quota=10 ** 6) + ["s_nop 7", "s_nop 7"] + self.split_tail(par)

    def pre_body(self):
        frags = self.qk_frags(0)
        ops = self.phase_a(0, True, earliest=2 * self.NDS + 2)
        return self.addr_k("s61") + self.schedule(frags, ops)

    def vm_wait_cases(self, sreg_count, cases, tag):
        out = []
        ends = self.label(tag + "e")
        for k in sorted(cases, reverse=True):
            if k == 0:
                out += ["s_waitcnt vmcnt(0)"]
            else:
                nxt = self.label(tag)
                out += [f"s_cmp_ge_u32 {sreg_count}, {k}", f"s_cbranch_scc0 {nxt}",
                        f"s_waitcnt vmcnt({self.NLD * k})", f"s_branch {ends}", f"{nxt}:"]
        out.append(f"{ends}:")
        return out

    def loop_top(self, last_label, par):
        """Even periods j: wait for this wave's share of blocks j+1 and j+2, barrier
        (every wave has finished period j-1, so the stages of blocks j-2 and j-1 are
        free), DMA pointers and exec masks for blocks j+3 and j+4.  Odd periods: no
        wait, barrier or DMA."""
        out = ["s_cmp_ge_u32 s58, s59", f"s_cbranch_scc1 {last_label}"]
        if par == 1:
            return out + [f"v_subrev_u32 {st('lim')}, 64, {st('lim')}"]
        # at j = 0 the prologue's blocks 3 .. min(nb, NS)-1 were issued after blocks 1, 2;
        # later, blocks j+1 and j+2 are the last ones issued (period j-2)
        w0, wd = self.label("wz"), self.label("wd")
        out += ["s_cmp_eq_u32 s58, 0", f"s_cbranch_scc0 {w0}",
                f"s_min_u32 s64, {o('nb')}, {NS}", "s_sub_u32 s64, s64, 3", "s_max_i32 s64, s64, 0"]
        out += self.vm_wait_cases("s64", list(range(NS - 2)), "wl")
        out += [f"s_branch {wd}", f"{w0}:", "s_waitcnt vmcnt(0)", f"{wd}:"]
        out += ["s_barrier"]
        skip = self.label("dsk")
        out += ["s_mov_b32 s62, s53", "s_mov_b32 s63, s54"] + self.rotate("s62") + ["s_add_u32 s63, s63, 64",
                "s_mov_b32 s53, s62", "s_mov_b32 s54, s63"] + self.rotate("s53") + ["s_add_u32 s54, s54, 64",
                "s_mov_b64 s[76:77], exec", "s_mov_b64 s[74:75], 0", "s_mov_b64 s[92:93], 0",
                "s_cmp_eq_u32 s58, 0", f"s_cbranch_scc1 {skip}",
                "s_add_u32 s64, s58, 3", f"s_cmp_ge_u32 s64, {o('nb')}", f"s_cbranch_scc1 {skip}",
                "s_mov_b64 s[74:75], exec",
                "s_add_u32 s64, s58, 4", f"s_cmp_ge_u32 s64, {o('nb')}", f"s_cbranch_scc1 {skip}",
                "s_mov_b64 s[92:93], exec", f"{skip}:",
                f"v_subrev_u32 {st('lim')}, 64, {st('lim')}"]
        return out

    def fin(self, par, last_label, drain):
        """Period j = jl of a wave whose last unmasked block jl is not the workgroup's
        last: PV(jl) with the period's DMA and barrier, without S(jl+1) (all masked);
        then the drain."""
        frags = self.pv_frags()
        npv = 4 * self.NDT
        ops = [dict(lines=g, deadline=min(12, npv - 2), earliest=-1) for g in
               (self.dma_lines(True) if par == 0 else self.dma_lines(True, "s53", "s54", "s[92:93]"))]
        ops += self.phase_b(par, pv0=0)
        body = self.schedule(frags, ops, pre_quota=10 ** 6)
        return (self.loop_top(last_label, par) + self.addr_v("s61") + body + ["s_nop 7", "s_nop 7"] +
                self.split_tail(par) + ["s_add_u32 s58, s58, 1", f"s_branch {drain[1 - par]}"])

    def drain(self, labels, epi):
        """Periods after the wave's last unmasked block: the same waits, barriers and
        DMA issues as the loop's periods (so every wave passes the same barriers and
        fills its share of the ring), no MFMA, softmax or LDS reads; the final PV
        block is skipped as well.  labels: entry at an even / odd period."""
        done = self.label("dlast")
        out = [f"{labels[0]}:"] + self.loop_top(done, 0)
        for g in self.dma_lines(True):
            out += g
        out += ["s_add_u32 s58, s58, 1", f"{labels[1]}:"] + self.loop_top(done, 1)
        for g in self.dma_lines(True, "s53", "s54", "s[92:93]"):
            out += g
        out += ["s_add_u32 s58, s58, 1", f"s_branch {labels[0]}", f"{done}:", f"s_branch {epi}"]
        return out

    def program(self):
        # m0 (the LDS address of the DMA loads) belongs to the compiler: it is saved
        # here and restored at the single exit, so the asm statement preserves it
        out = ["s_mov_b32 s52, m0", f"v_mov_b32 {NINF}, 0xff800000"]
        out += [f"v_mov_b32 v{O_BASE + k}, 0" for k in range(16 * self.NDT)]
        for ds in range(self.NDS):
            q0 = Q_BASE + 4 * ds
            out.append(f"global_load_dwordx4 {vr(q0, q0 + 3)}, {o('qp')}, off offset:{32 * ds}")
        out += [f"v_mov_b32 {st('m')}, {NINF}", f"v_mov_b32 {st('l')}, 0", f"v_mov_b32 {st('lim')}, {o('lim')}"]
        out += ["s_mov_b64 s[48:49], " + o("kbase"), "s_mov_b64 s[56:57], " + o("vbase")]
        out += [f"s_add_u32 s65, {o('lds')}, {NS * self.SS}"]
        out += [f"s_mov_b32 s62, {o('lds')}", "s_mov_b32 s63, 0"]
        for s in range(NS):
            skip = self.label("pd")
            out += [f"s_cmp_lt_u32 {s}, {o('nb')}", f"s_cbranch_scc0 {skip}"]
            for g in self.dma_lines(False):
                out += g
            out += [f"{skip}:", f"s_add_u32 s62, s62, {self.SS}", "s_add_u32 s63, s63, 64"]
        out += [f"s_min_u32 s64, {o('nb')}, {NS}", "s_sub_u32 s64, s64, 1"]
        out += self.vm_wait_cases("s64", list(range(NS)), "w0")
        out += ["s_barrier"]
        out += [f"s_mov_b32 s61, {o('lds')}", f"s_add_u32 s60, {o('lds')}, {self.SS}",
                f"s_add_u32 s53, {o('lds')}, {2 * self.SS}", "s_mov_b32 s54, 128",
                "s_mov_b32 s58, 0", f"s_sub_u32 s59, {o('nb')}, 1"]
        out += self.pre_body()
        top = [self.label("top0"), self.label("top1")]
        last = [self.label("last0"), self.label("last1")]
        epi = self.label("epi")
        drain = [self.label("drain0"), self.label("drain1")]
        fin = [self.label("fin0"), self.label("fin1")]
        for par in (0, 1):
            msk, nxt = self.label("msk"), self.label("nxt")
            # past the wave's last block (jl) every score is masked: only the ring
            # duties (DMA share, barrier) remain
            out += [f"{top[par]}:", f"s_cmp_gt_u32 s58, {o('jl')}", f"s_cbranch_scc1 {drain[par]}",
                    f"s_cmp_eq_u32 s58, {o('jl')}", f"s_cbranch_scc1 {fin[par]}"]
            out += self.loop_top(last[par], par)
            out += ["s_add_u32 s64, s58, 1", f"s_cmp_ge_u32 s64, {o('jd')}", f"s_cbranch_scc1 {msk}"]
            out += self.period(par, False)
            out += [f"s_branch {nxt}", f"{msk}:"]
            out += self.period(par, True)
            out += [f"{nxt}:"] + self.rotate("s60") + self.rotate("s61") + ["s_add_u32 s58, s58, 1"]
        out += [f"s_branch {top[0]}"]
        for par in (0, 1):
            out += [f"{last[par]}:"]
            out += self.last(par) + [f"s_branch {epi}"]
        for par in (0, 1):
            out += [f"{fin[par]}:"] + self.fin(par, last[par], drain)
        out += self.drain(drain, epi)
        out += [f"{epi}:", "s_waitcnt lgkmcnt(0)", "s_nop 7", "s_nop 7", "s_nop 7",
                "s_mov_b64 s[66:67], exec"]
        out += [f"v_mov_b32 v32, {st('l')}", f"v_mov_b32 v33, {st('l')}", "s_nop 1",
                "v_permlane32_swap_b32 v32, v33", "s_nop 1",
                "v_add_f32 v32, v32, v33"]
        if self.partial:
            # Split-KV part: the unnormalized O row in f32 (this lane's 64 values, 4 at a
            # time: d = 32 dtl + 8 q4 + 4 g + 0..3), then {l, m} after the 128 values,
            # written by the lanes of half 0 (op = record + 16 g bytes).
            out += [f"v_mov_b32 v33, {st('m')}", f"s_mov_b64 exec, {o('ok')}"]
            for dtl in range(self.NDT):
                for q4 in range(4):
                    a = O_BASE + 16 * dtl + 4 * q4
                    out.append(f"global_store_dwordx4 {o('op')}, v[{a}:{a + 3}], off offset:{128 * dtl + 32 * q4}")
            out += ["s_mov_b32 exec_hi, 0", f"global_store_dwordx2 {o('op')}, v[32:33], off offset:{4 * self.D}"]
        else:
            out += ["v_rcp_f32 v34, v32", "s_nop 0", f"s_mov_b64 exec, {o('ok')}"]
            for dtl in range(self.NDT):
                for q4 in range(4):
                    a = O_BASE + 16 * dtl + 4 * q4
                    out += [f"v_mul_f32 v{36 + k}, v34, v{a + k}" for k in range(4)]
                    out += [f"{self.cvt} v40, v36, v37", f"{self.cvt} v41, v38, v39",
                            f"global_store_dwordx2 {o('op')}, v[40:41], off offset:{64 * dtl + 16 * q4}"]
        out += ["s_mov_b64 exec, s[66:67]"]
        end = self.label("end")
        out += [f"s_branch {end}"]
        for blk in self.ool:
            out += blk
        out += [f"{end}:", "s_waitcnt vmcnt(0)", "s_mov_b32 m0, s52"]
        return out


def cstr(lines):
    return "\\n\\t".join(lines)


def main(path):
    lines = ["// Generated by gen_prefill.py: prefill main loop (gfx950 asm).", "#pragma once"]
    for d in (128, 64):
        for dt in ("bf16", "f16"):
            for partial in (False, True):
                prog = Gen(dt, partial, d).program()
                name = dt.upper() + ("_PART" if partial else "") + ("" if d == 128 else "_D64")
                lines.append(f'#define TH_PREFILL_ASM_{name} "{cstr(prog)}"')
    clob = [f'"v{k}"' for k in range(16, 256)] + [f'"s{k}"' for k in range(48, 96)]
    lines.append("#define TH_PREFILL_ASM_CLOBBERS " + ",".join(clob))
    text = "\n".join(lines) + "\n"
    p = Path(path)
    if not p.exists() or p.read_text() != text:
        p.parent.mkdir(parents=True, exist_ok=True)
        p.write_text(text)


if __name__ == "__main__":
    main(sys.argv[1])
