"""Generate the dense 16-bit GEMM tile program (gfx950 assembly for one inline-asm
statement; gemm_asm.hpp wraps it).

Semantics: C = A . B with f32 accumulation (`linalg.fill 0` + `linalg.matmul`,
/root/reference/crates/rustc_codegen_tile/src/mlir_to_linalg.rs:1345-1393), A row-major
M x K, B row-major K x N, bf16 or f16 operands, C f32 or 16-bit (one rounding, RNE).

Workgroup = 4 waves = one 256 x 256 tile; wave (wm, wn) = (w / 2, w % 2) owns rows
128 wm .. +127 and columns 128 wn .. +127 as 8 x 8 blocks of 16 x 16, accumulated in
a[0:255] (block (mi, ni) at a[4 (8 mi + ni)]) with v_mfma_f32_16x16x32, one MFMA per
block and 32-deep K step.  One wave per SIMD: the 128 x 128 wave tile reads 64 KB of
LDS fragments per K step for the workgroup, a third less than eight waves of 128 x 64.
The 16x16x32 form moves half the accumulator data of 32x32x16 per FLOP; the chip runs
power-limited, and on random operands the same MFMA work takes 62.8-68.4 us instead of
73.0-78.2 us (microbenchmark, 4096 x 32768 FLOP per SIMD).  Both forms round the same
way here: C is bit-identical to the 32x32x16 program on both config shapes.

K advances 32 per step.  LDS (128 KB), filled by global_load_lds_dwordx4 only:
  A ring: 2 double stages x 32 KB at 0.  A double stage holds 64 k of the tile's 256
          rows, [256 r][8 chunks of 16 B]: every DMA lane group reads whole 128-byte
          rows of A (with 32-k stages each row would be half a cache line).  Chunk c
          of row r sits at c ^ (r & 7): conflict-free for the fragment reads (16 rows
          x 4 chunks per instruction), where (r & 7) ^ ((r >> 3) & 1) measured 2-way
          bank conflicts and no swizzle 4-way (SQ_LDS_BANK_CONFLICT, probe of the
          lane pattern).
  B ring: 4 stages x 16 KB at 64 KB, [32 k][32 chunks]: chunk c of k-row r at
          c ^ sb(r), sb(r) = 4 (r & 3) ^ 2 ((r >> 3) & 1); read as B^T with
          ds_read_b64_tr_b16.  A transposed read covers 32 lanes per cycle: the two
          16-lane groups read k rows 8 apart, and bit 3 of the row in sb keeps their
          16 chunks apart (without it the B reads took 2-way bank conflicts in half of
          the LDS-active cycles).
Step k uses A double stage k/2 (buffer (k/2) % 2, k half k % 2) and B stage k
(buffer k % 4).

B stored N x K (`bt`, the transposed matmul): B^T rows are K-contiguous like A's, so
B takes A's form: a ring of 2 double stages x 32 KB at 64 KB ([256 n][8 chunks],
chunk c of row n at c ^ (n & 7)), read with ds_read_b128 like A, and refilled at the
same odd steps.  Then the only wait is at odd k, for double stage (k+1)/2 of both
operands, which nothing has been issued after (vmcnt(0)); it was issued two steps
earlier.  The prologue issues A0, B0, A1, B1 and waits for A0, B0 (vmcnt(16)).

Schedule of step k (every wave):
  s_waitcnt lgkmcnt(0)        this wave's fragments of step k have landed
  s_waitcnt vmcnt(n)          this wave's DMA share of B stage k+1 and of A double
                              stage (k+1)/2 has landed (n: loads issued after them)
  s_barrier                   -> every share of those stages is in LDS, and every
                              wave has finished reading step k's fragments
  64 MFMAs of step k, with in between: the 24 fragment reads of step k+1 (into the
  other register set, one after every second MFMA from the first) and the DMA issues:
  B stage k+4 into buffer k % 4 (free: step k's reads are done) and, at odd k, A
  double stage (k+3)/2 into buffer ((k+3)/2) % 2 (free: its last reader, step k, is
  done).
Per-wave issue order, steady state: even k: B(k+4); odd k: A((k+3)/2), B(k+4).  At
the wait of even k the loads issued after B(k+1) are B(k+2), A(k/2+1), B(k+3) (16);
at odd k those after A((k+1)/2) are B(k+2), B(k+3) (8).  The prologue issues B0, A0,
B1, B2, A1, B3, which is the same sequence, so the steady waits hold from step 0.  A
double stage is issued two steps before its first reader, a B stage three.  The loop
runs in groups of four steps (static buffers); the last group issues no DMA and waits
16, 4, 0.

Fragments of a step: A block mi (16 rows x 32 k): lane l reads row 16 mi + l % 16,
the 16 bytes of k 8 (l / 16) .. +7 (ds_read_b128); B block ni (32 k x 16 columns):
lane l needs column 16 ni + l % 16 at k 8 (l / 16) .. +7, two ds_read_b64_tr_b16 of
four k rows each.

Registers: operands in v0-v15 and s-registers chosen by the compiler; v16-v17 A read
bases [h], v52-v59 B read bases [ni], v24-v31 A DMA offsets,
v32-v51 epilogue, v[128:191] and v[192:255] the two fragment sets (A mi at +4 mi, B ni
at +32 + 4 ni); s[48:49] A pointer, s[50:51] B pointer, s[52:53] C base, s54 loop
count, s55 saved m0, s56-s57 temps.

SiLU*Mul form (C = silu(A.B) * UP, 16-bit C and UP): the same loop; the last step opens
with a barrier (every wave has read its last fragments), after which each wave DMAs its
128 x 128 UP tile into its own 32 KB of the idle ring under the last step's MFMAs
(s[58:59] the UP pointer), waits for it (no store has been issued yet, so vmcnt(0)
covers exactly the UP loads), and runs epilogue_silu.  v[128:135] are its temps.

Usage: python gen_gemm.py <out.inc>   (run by the library build)
"""
import sys
from pathlib import Path

OPN = ["aoffE", "aoffO", "boff0", "boff1", "boff2", "boff3", "ra0", "ra1",
       "rb0", "rb1", "rb2", "rb3", "coff",
       "abase", "bbase", "cbase", "nk", "lds", "ldsa", "ldsb", "bstep", "nstride", "arow8",
       # the SiLU*Mul program only: UP tile base, wave's LDS staging region (m0 of the UP
       # DMA), per-lane UP DMA offset, per-lane LDS read base
       "ubase", "ustage", "uoff", "uread"]
OP = {n: i for i, n in enumerate(OPN)}


def o(n):
    return f"%{OP[n]}"


SA_, SB_, SC_ = "s[48:49]", "s[50:51]", "s[52:53]"
SCNT, SROW = "s54", "s57"
VA = [16, 17]                    # A read bases [h]
VB = list(range(52, 60))         # B read bases [ni]
VAO = list(range(24, 32))        # A DMA offsets, unit j = 0..7
VBO = list(range(60, 68))        # B DMA offsets (bt), unit j = 0..7
BT = [False]                     # the program being generated has B stored N x K
FR = [128, 192]                  # fragment register sets


def afr(s, mi):
    return FR[s] + 4 * mi


def bfr(s, ni):
    return FR[s] + 32 + 4 * ni


def acc(mi, ni):
    b = 4 * (8 * mi + ni)
    return f"a[{b}:{b + 3}]"


def reads(k, s):
    """Fragment reads of step k (mod 4) into register set s: A (8 blocks of 16 rows,
    16 bytes per lane), then B^T (8 blocks of 16 columns, two transposed 8-byte reads
    each)."""
    ab, h, bb = (k // 2) % 2, k % 2, k % 4
    out = []
    for mi in range(8):
        f = afr(s, mi)
        out.append(f"ds_read_b128 v[{f}:{f + 3}], v{VA[h]} offset:{ab * 32768 + 2048 * mi}")
    if BT[0]:
        for ni in range(8):
            f = bfr(s, ni)
            out.append(f"ds_read_b128 v[{f}:{f + 3}], v{VB[h]} offset:{ab * 32768 + 2048 * ni}")
        return out
    for ni in range(8):
        f = bfr(s, ni)
        base = bb * 16384
        out.append(f"ds_read_b64_tr_b16 v[{f}:{f + 1}], v{VB[ni]} offset:{base}")
        out.append(f"ds_read_b64_tr_b16 v[{f + 2}:{f + 3}], v{VB[ni]} offset:{base + 2048}")
    return out


def dma_b(buf):
    """This wave's four 1 KB units of the next B stage into buffer buf (bt: eight units
    of the next B double stage, like A).  The LDS destination (m0) needs one wait state
    after it is written."""
    out = []
    if BT[0]:
        for j in range(8):
            out.append([f"s_add_u32 m0, {o('ldsb')}, {buf * 32768 + j * 1024}", "s_nop 0",
                        f"global_load_lds_dwordx4 v{VBO[j]}, {SB_}"])
        out.append(["s_add_u32 s50, s50, 128", "s_addc_u32 s51, s51, 0"])
        return out
    for j in range(4):
        out.append([f"s_add_u32 m0, {o('ldsb')}, {buf * 16384 + j * 1024}", "s_nop 0",
                    f"global_load_lds_dwordx4 {o('boff' + str(j))}, {SB_}"])
    out.append([f"s_add_u32 s50, s50, {o('bstep')}", "s_addc_u32 s51, s51, 0"])
    return out


def dma_a(buf):
    """This wave's eight 1 KB units (8 rows x 128 B each) of the next A double stage."""
    out = []
    for j in range(8):
        out.append([f"s_add_u32 m0, {o('ldsa')}, {buf * 32768 + j * 1024}", "s_nop 0",
                    f"global_load_lds_dwordx4 v{VAO[j]}, {SA_}"])
    out.append(["s_add_u32 s48, s48, 128", "s_addc_u32 s49, s49, 0"])
    return out


def mfmas(s, mn):
    """The step's 64 MFMAs, row block by row block, the column order reversed on odd rows
    (each row's A fragment, and one B fragment across the turn, feed consecutive MFMAs;
    0.6 us less at 4096^3 than the same order on every row)."""
    out = []
    for mi in range(8):
        for ni in (range(8) if mi % 2 == 0 else range(7, -1, -1)):
            a, b = afr(s, mi), bfr(s, ni)
            out.append(f"{mn} {acc(mi, ni)}, v[{a}:{a + 3}], v[{b}:{b + 3}], {acc(mi, ni)}")
    return out


DEFER = 4   # MFMAs of each step issued after the next step's barrier


def deferred(k4, mn):
    """The last DEFER MFMAs of step k4: issued after the next step's waits and barrier,
    they keep the MFMA pipe busy while the barrier resolves.  They read only registers
    already loaded, and the next reads into their fragment set are issued after them."""
    return mfmas(k4 & 1, mn)[64 - DEFER:]


def step(k4, mn, vm, rd, dm, bar=True, carry=(), defer=True):
    """Step k with k % 4 == k4: waits, barrier, the previous step's deferred MFMAs
    (`carry`), then this step's MFMAs (all but the deferred ones when `defer`).  The
    reads of step k+1 go one after every second MFMA of the first 48 (measured at
    4096^3 against 12, 24 and 64 MFMAs: 1-7 us less); the DMA groups start after the
    first MFMA and spread over the step."""
    out = ["s_waitcnt lgkmcnt(0)"]
    if vm is not None:
        out.append(f"s_waitcnt vmcnt({vm})")
    if bar:
        out.append("s_barrier")
    out += list(carry)
    M = mfmas(k4 & 1, mn)
    if defer:
        M = M[:64 - DEFER]
    R = reads((k4 + 1) % 4, (k4 + 1) & 1) if rd else []
    D = []
    if dm:
        if k4 % 2 == 1:
            D += dma_a(((k4 + 3) // 2) % 2)
            if BT[0]:
                D += dma_b(((k4 + 3) // 2) % 2)
        if not BT[0]:
            D += dma_b(k4)
    slots = [[] for _ in M]
    for j, r in enumerate(R):
        slots[2 * j].append([r])
    for j, d in enumerate(D):
        slots[min(len(M) - 1, (j * len(M)) // len(D) + 1)].append(d)
    for m, sl in zip(M, slots):
        out.append(m)
        for g in sl:
            out.extend(g)
    return out


def epilogue(out_dt, mis=range(8)):
    """C stores from the accumulators.  Accumulator r of lane l in a 16x16 block is row
    4 (l / 16) + r, column l % 16, so a store straight from one block writes 64-byte row
    pieces.  For each row r and pair of column blocks (2p, 2p+1) the two values go
    through v_permlane16_swap: afterwards one register holds rows r and 8 + r, the other
    rows 4 + r and 12 + r, each with lane l at column 32 p + l % 32, so one store
    writes two rows of 32 columns (f32: whole 128-byte lines; 5.5 us less than the
    direct stores at 4096^3, same bits).  16-bit C packs rows r, r+1 first
    (v_cvt_pk_{bf16,f16}_f32, RNE) and writes them with short / short_d16_hi stores.
    coff = this lane's byte offset (row 8 (l / 32), column l % 32)."""
    L = []
    if out_dt == "f32":
        for mi in mis:
            for r in range(4):
                row = mi * 16 + r
                L.append(f"s_mul_i32 {SROW}, {o('nstride')}, {row}")
                L.append(f"v_add_u32 v32, {SROW}, {o('coff')}")
                L.append(f"s_lshl_b32 s56, {o('nstride')}, 2")
                L.append("v_add_u32 v33, s56, v32")
                for ni in range(8):
                    L.append(f"v_accvgpr_read_b32 v{36 + ni}, a{4 * (8 * mi + ni) + r}")
                L.append("s_nop 1")
                for p in range(4):
                    L.append(f"v_permlane16_swap_b32 v{36 + 2 * p}, v{37 + 2 * p}")
                L.append("s_nop 1")
                for p in range(4):
                    L.append(f"global_store_dword v32, v{36 + 2 * p}, {SC_} offset:{128 * p} nt")
                    L.append(f"global_store_dword v33, v{37 + 2 * p}, {SC_} offset:{128 * p} nt")
        return L
    cvt = "v_cvt_pk_bf16_f32" if out_dt == "bf16" else "v_cvt_pk_f16_f32"
    for mi in mis:
        for r in range(0, 4, 2):
            row = mi * 16 + r     # rows row, row + 1 (and + 4, + 5 after the swap)
            L.append(f"s_mul_i32 {SROW}, {o('nstride')}, {row}")
            L.append(f"v_add_u32 v32, {SROW}, {o('coff')}")
            L.append(f"v_add_u32 v33, {o('nstride')}, v32")
            L.append(f"s_lshl_b32 s56, {o('nstride')}, 2")
            L.append("v_add_u32 v34, s56, v32")
            L.append("v_add_u32 v35, s56, v33")
            for ni in range(8):
                a = 4 * (8 * mi + ni) + r
                t = 36 + 2 * ni
                L += [f"v_accvgpr_read_b32 v{t}, a{a}", f"v_accvgpr_read_b32 v{t + 1}, a{a + 1}",
                      f"{cvt} v{t}, v{t}, v{t + 1}"]
            L.append("s_nop 1")
            for p in range(4):
                L.append(f"v_permlane16_swap_b32 v{36 + 4 * p}, v{38 + 4 * p}")
            L.append("s_nop 1")
            for p in range(4):
                x, y = 36 + 4 * p, 38 + 4 * p
                L += [f"global_store_short v32, v{x}, {SC_} offset:{64 * p} nt",
                      f"global_store_short_d16_hi v33, v{x}, {SC_} offset:{64 * p} nt",
                      f"global_store_short v34, v{y}, {SC_} offset:{64 * p} nt",
                      f"global_store_short_d16_hi v35, v{y}, {SC_} offset:{64 * p} nt"]
    return L


LOG2E_NEG = "0xbfb8aa3b"   # -log2(e) in f32


def dma_up():
    """The SiLU*Mul program's UP tile: 32 units of four 256-byte rows (the wave's 128 rows
    x 128 columns, 16-bit) into the wave's 32 KB staging region, row-major."""
    out = [[f"s_mov_b64 s[58:59], {o('ubase')}", f"s_lshl_b32 s56, {o('nstride')}, 2"]]
    for j in range(32):
        out.append([f"s_add_u32 m0, {o('ustage')}, {1024 * j}", "s_nop 0",
                    f"global_load_lds_dwordx4 {o('uoff')}, s[58:59]",
                    "s_add_u32 s58, s58, s56", "s_addc_u32 s59, s59, 0"])
    return out


def epilogue_silu(out_dt):
    """C = silu(acc) * UP for 16-bit C, silu(x) = x / (1 + exp(-x)) as x * rcp(1 +
    2^(-x log2 e)) in f32 (v_exp_f32, v_rcp_f32), one rounding at the end.  Values go
    through the same lane swap as the f32 stores; UP comes from the staging region at
    the same (row, column) and C is written with short stores (two rows of 32 columns
    per store)."""
    cvt = "v_cvt_pk_bf16_f32" if out_dt == "bf16" else "v_cvt_pk_f16_f32"
    T = list(range(128, 136))     # temps: fragment registers, free after the last MFMAs
    L = [f"s_lshl_b32 s56, {o('nstride')}, 2"]
    for mi in range(8):
        for r in range(4):
            row = mi * 16 + r
            L.append(f"s_mul_i32 {SROW}, {o('nstride')}, {row}")
            L.append(f"v_add_u32 v32, {SROW}, {o('coff')}")
            L.append("v_add_u32 v33, s56, v32")
            for ni in range(8):
                L.append(f"v_accvgpr_read_b32 v{36 + ni}, a{4 * (8 * mi + ni) + r}")
            for p in range(4):
                L.append(f"ds_read_u16 v{44 + 2 * p}, {o('uread')} offset:{256 * row + 64 * p}")
                L.append(f"ds_read_u16 v{45 + 2 * p}, {o('uread')} offset:{256 * (row + 4) + 64 * p}")
            L.append("s_nop 1")
            for p in range(4):
                L.append(f"v_permlane16_swap_b32 v{36 + 2 * p}, v{37 + 2 * p}")
            L.append("s_nop 1")
            G, U = [36 + k for k in range(8)], [44 + k for k in range(8)]
            for k in range(8):
                L.append(f"v_mul_f32 v{T[k]}, {LOG2E_NEG}, v{G[k]}")
            for k in range(8):
                L.append(f"v_exp_f32 v{T[k]}, v{T[k]}")
            for k in range(8):
                L.append(f"v_add_f32 v{T[k]}, 1.0, v{T[k]}")
            for k in range(8):
                L.append(f"v_rcp_f32 v{T[k]}, v{T[k]}")
            for k in range(8):
                L.append(f"v_mul_f32 v{T[k]}, v{G[k]}, v{T[k]}")
            L.append("s_waitcnt lgkmcnt(0)")
            for k in range(8):
                if out_dt == "bf16":
                    L.append(f"v_lshlrev_b32 v{U[k]}, 16, v{U[k]}")
                else:
                    L.append(f"v_cvt_f32_f16 v{U[k]}, v{U[k]}")
            for k in range(8):
                L.append(f"v_mul_f32 v{G[k]}, v{T[k]}, v{U[k]}")
            for k in range(8):
                L.append(f"{cvt} v{G[k]}, v{G[k]}, v{G[k]}")
            for p in range(4):
                L.append(f"global_store_short v32, v{36 + 2 * p}, {SC_} offset:{64 * p} nt")
                L.append(f"global_store_short v33, v{37 + 2 * p}, {SC_} offset:{64 * p} nt")
    return L


def vm(k4, steady):
    """vmcnt of step k % 4 == k4 (None: no wait), steady: the group issues DMA."""
    if BT[0]:
        return 0 if k4 % 2 == 1 else None
    if steady:
        return 16 if k4 % 2 == 0 else 8
    return [16, 4, 0, None][k4]


def program(dt, out_dt, bt=False, silu=False):
    """silu: the SiLU*Mul epilogue (16-bit C): after the barrier that opens the last
    step, when every wave has read its last fragments, each wave's UP tile is fetched
    into its 32 KB of the (then idle) ring under the last step's MFMAs."""
    assert not silu or out_dt != "f32"
    BT[0] = bt
    mn = "v_mfma_f32_16x16x32_bf16" if dt == "bf16" else "v_mfma_f32_16x16x32_f16"
    L = ["s_mov_b32 s55, m0",
         f"s_mov_b64 {SA_}, {o('abase')}", f"s_mov_b64 {SB_}, {o('bbase')}",
         f"s_mov_b64 {SC_}, {o('cbase')}"]
    for h in range(2):
        L.append(f"v_add_u32 v{VA[h]}, {o('lds')}, {o('ra' + str(h))}")
    if bt:
        # B^T read bases [h] (rb0, rb1), DMA offsets like A's (boff0, boff1 = units 0, 1)
        for h in range(2):
            L += [f"v_add_u32 v{VB[h]}, {o('lds')}, {o('rb' + str(h))}",
                  f"v_add_u32 v{VB[h]}, 0x10000, v{VB[h]}"]
        for j in range(8):
            L.append(f"s_mul_i32 {SROW}, {o('arow8')}, {j & ~1}")
            L.append(f"v_add_u32 v{VBO[j]}, {SROW}, {o('boff' + str(j & 1))}")
    else:
        # block 2p + 1 is 16 columns on: chunk bit 1 flips (bytes ^ 32), whatever sb adds
        for p in range(4):
            ev, od = VB[2 * p], VB[2 * p + 1]
            L += [f"v_add_u32 v{ev}, {o('lds')}, {o('rb' + str(p))}", f"v_add_u32 v{ev}, 0x10000, v{ev}",
                  f"v_xor_b32 v{od}, 32, {o('rb' + str(p))}", f"v_add_u32 v{od}, {o('lds')}, v{od}",
                  f"v_add_u32 v{od}, 0x10000, v{od}"]
    # A unit j of wave w holds rows 64 w + 8 j .. +7: units j and j & 1 differ by
    # (j & ~1) x 8 rows (the swizzle depends on the row's low three bits only)
    for j in range(8):
        src = o("aoffE") if j % 2 == 0 else o("aoffO")
        L.append(f"s_mul_i32 {SROW}, {o('arow8')}, {j & ~1}")
        L.append(f"v_add_u32 v{VAO[j]}, {SROW}, {src}")
    L += [f"v_accvgpr_write_b32 a{r}, 0" for r in range(256)]
    if bt:
        for g in dma_a(0) + dma_b(0) + dma_a(1) + dma_b(1):
            L.extend(g)
        # A0 and B0 landed: loads issued after B0 are A1, B1 (8 + 8)
        L += ["s_waitcnt vmcnt(16)", "s_barrier"] + reads(0, 0)
    else:
        for g in dma_b(0) + dma_a(0) + dma_b(1) + dma_b(2) + dma_a(1) + dma_b(3):
            L.extend(g)
        # B0 and A0 landed: loads issued after A0 are B1, B2, A1, B3 (4 + 4 + 8 + 4)
        L += ["s_waitcnt vmcnt(20)", "s_barrier"] + reads(0, 0)
    # steady groups: nk / 4 - 1 (nk >= 8, a multiple of 4: checked by the caller; a
    # launch outside that would skip the work and write nothing).  The first group
    # enters at its step 1 after a copy of step 0 with nothing carried in.
    L += [f"s_lshr_b32 {SCNT}, {o('nk')}, 2", f"s_sub_u32 {SCNT}, {SCNT}, 1",
          f"s_cmp_eq_u32 {SCNT}, 0", "s_cbranch_scc1 L_end_%="]
    L += step(0, mn, vm(0, True), True, True) + ["s_branch L_b1_%="]
    L += ["L_top_%=:"] + step(0, mn, vm(0, True), True, True, carry=deferred(3, mn))
    L += ["L_b1_%=:"]
    for k4 in (1, 2, 3):
        L += step(k4, mn, vm(k4, True), True, True, carry=deferred(k4 - 1, mn))
    L += [f"s_sub_u32 {SCNT}, {SCNT}, 1", f"s_cmp_lg_u32 {SCNT}, 0", "s_cbranch_scc1 L_top_%="]
    for k4 in (0, 1, 2):
        L += step(k4, mn, vm(k4, False), True, False, carry=deferred((k4 + 3) % 4, mn))
    # the last step: row block mi's stores start once the MFMAs of row block mi + 2
    # have issued (16 MFMAs after its last one: its results are written), the last
    # two row blocks' after the loop
    if silu:
        L += ["s_waitcnt lgkmcnt(0)", "s_barrier"] + deferred(2, mn)
        M = mfmas(1, mn)
        D = dma_up()
        slots = [[] for _ in M]
        for j, d in enumerate(D):
            slots[min(len(M) - 1, (j * len(M)) // len(D))].append(d)
        for m, sl in zip(M, slots):
            L.append(m)
            for g in sl:
                L.extend(g)
        # MFMA results -> readers; UP landed (no store issued yet)
        L += ["s_nop 7", "s_nop 7", "s_nop 7", "s_nop 7", "s_waitcnt vmcnt(0)"]
        L += epilogue_silu(out_dt)
    else:
        L += ["s_waitcnt lgkmcnt(0)"] + deferred(2, mn)
        M = mfmas(1, mn)
        for mi in range(8):
            L += M[8 * mi:8 * mi + 8]
            if mi >= 2:
                L += epilogue(out_dt, [mi - 2])
        L += ["s_nop 7", "s_nop 7", "s_nop 7", "s_nop 7"]   # MFMA results -> readers
        L += epilogue(out_dt, [6, 7])
    L += ["L_end_%=:"]
    L += ["s_waitcnt vmcnt(0)", "s_mov_b32 m0, s55"]
    return L


def cstr(lines):
    return "\\n\\t".join(lines)


def main(path):
    lines = ["// Generated by gen_gemm.py: 16-bit GEMM tile program (gfx950 asm).", "#pragma once"]
    for bt in (False, True):
        for dt in ("bf16", "f16"):
            for out_dt in ("f32", "bf16", "f16"):
                lines.append(f'#define TH_GEMM_ASM_{dt.upper()}_{out_dt.upper()}{"_BT" if bt else ""} '
                             f'"{cstr(program(dt, out_dt, bt))}"')
    for bt in (False, True):
        for dt in ("bf16", "f16"):
            for out_dt in ("bf16", "f16"):
                lines.append(f'#define TH_GEMM_ASM_SILU_{dt.upper()}_{out_dt.upper()}{"_BT" if bt else ""} '
                             f'"{cstr(program(dt, out_dt, bt, silu=True))}"')
    clob = ([f'"v{k}"' for k in range(16, 256)] + [f'"a{k}"' for k in range(256)] +
            [f'"s{k}"' for k in range(48, 58)])
    lines.append("#define TH_GEMM_ASM_CLOBBERS " + ",".join(clob))
    lines.append("#define TH_GEMM_ASM_SILU_CLOBBERS TH_GEMM_ASM_CLOBBERS, \"s58\", \"s59\"")
    text = "\n".join(lines) + "\n"
    p = Path(path)
    if not p.exists() or p.read_text() != text:
        p.parent.mkdir(parents=True, exist_ok=True)
        p.write_text(text)


if __name__ == "__main__":
    main(sys.argv[1])
