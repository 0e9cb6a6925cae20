// Attention kernels: causal GQA prefill (flash, MFMA), GQA decode (split-KV,
// MFMA scores), and a general online-softmax kernel for every other shape/dtype.
//
// Semantics (reference):
//   prefill  __tile_attention_prefill_f32  crates/tile_std/src/tile.rs:2136, :3064;
//            Metal template mlir_to_msl.rs:10928-11009, host params :1851-1859.
//            query qi of head h sits at absolute position start_pos + qi and sees
//            KV positions pos <= start_pos + qi of kv_head = h / (NH / NKV);
//            scale = rsqrt(D).
//   decode   __tile_attention_decode_f32   tile.rs:2124, :3011; mlir_to_msl.rs:
//            10747-10816, host params :1816-1823: one query per head, positions
//            [0, seq_len), same GQA map and scale.
//   single   __tile_attention_f32          tile.rs:221, :2401; linalg
//            decomposition mlir_to_linalg.rs:1781-1902 (non-causal, one head,
//            scale 1/sqrt(D) computed in f64 then rounded to f32).
// Layouts in HBM: Q, O = [B][S][NH][D]; K, V = [B][NKV][max_seq][D] (the Metal
// templates' per-batch layout, stacked over the batch).  The Metal templates cap
// the KV length at 256; these kernels have no cap.
#pragma once

#include "common.hpp"
#include "gemm.hpp"

namespace th {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Hardware round-to-nearest-even packing of two floats (v_cvt_pk_bf16_f32 on gfx950).
template <int DT>
__device__ __forceinline__ uint32_t cvt_pk(float lo, float hi) {
  if constexpr (DT == kBF16) {
    bf16x2 v = __builtin_convertvector(f32x2{lo, hi}, bf16x2);
    return __builtin_bit_cast(uint32_t, v);
  } else {
    f16x2 v = __builtin_convertvector(f32x2{lo, hi}, f16x2);
    return __builtin_bit_cast(uint32_t, v);
  }
}

// ============================================================================
// Prefill: flash attention forward, causal, GQA, head_dim 128.
//
// Workgroup = 8 waves = 256 query rows of one (batch, head); wave w owns rows
// [32w, 32w+32).  KV is consumed 64 positions at a time.  Per wave and KV block:
//   S^T (64 kv x 32 q)  = K . Q^T          2x8 v_mfma_f32_32x32x16, Q^T in registers
//   online softmax on S^T columns: lane l owns query l%32; its partner lane l^32
//   holds the other half of that column, so row statistics need one exchange.
//   O^T (128 d x 32 q) += V^T . P^T        4x4 MFMAs; P^T is the S^T accumulator
//   converted to 16-bit in place: accumulator j of lane l (half g = l/32) is KV
//   row 8*(j/4) + 4g + j%4, and the V^T operand is read in the same KV order, so
//   the B operand needs no data movement.
// ============================================================================
namespace fa {
constexpr int D = 128;
constexpr int BQ = 256;   // query rows per workgroup
constexpr int NT = 512;   // threads per workgroup (8 waves)
constexpr float kRescaleThreshold = 8.0f;  // log2 units; see the rescale below
// A KV block whose probability mass exceeds 1/ratio of the query's running sum
// gets its P residual as well (bf16 keeps 8 significant bits, f16 keeps 11).
template <int DT> constexpr float kSplitRatio = (DT == kBF16) ? 16.0f : 2.0f;
}  // namespace fa

// Widen a packed pair of 16-bit values.
template <int DT>
__device__ __forceinline__ void unpack_pair(uint32_t d, float& lo, float& hi) {
  lo = u16_to_f32<DT>(static_cast<uint16_t>(d & 0xffffu));
  hi = u16_to_f32<DT>(static_cast<uint16_t>(d >> 16));
}

// Map a work index to (bh, qb): heavy (late) query blocks first; when the head
// count allows, heads are dealt to XCDs so one head's query blocks share an L2.
__device__ __forceinline__ void prefill_work(uint32_t w, uint32_t nbh, uint32_t nqb,
                                             uint32_t& bh, uint32_t& qb) {
  if (nbh % 8 == 0) {
    const uint32_t xcd = w % 8, r = w / 8, per = nbh / 8;
    bh = xcd + 8 * (r % per);
    qb = nqb - 1 - r / per;
  } else {
    bh = w % nbh;
    qb = nqb - 1 - w / nbh;
  }
}

// ============================================================================
// Prefill, LDS-DMA form (head_dim 128, 16-bit Q/K/V).
//
// The work split and arithmetic above (8 waves x 32 query rows, S^T = K.Q^T,
// online softmax per query column, O^T += V^T.P^T with P^T taken from the S^T
// accumulators in place).  K and V reach LDS by global_load_lds_dwordx4 into a
// ring of NS stages of 64 KV positions, issued NS-1 blocks ahead, with no
// register staging and no transpose on the way in:
//   K stage [64 kv][128 d]: 16-byte chunk c of row r at unit c ^ (r & 15), so
//            the 16 rows one quarter-wave reads with ds_read_b128 cover all 64
//            banks.
//   V stage [64 kv][128 d] row-major: chunk c of row r at unit c ^ 4*(r & 3).
//            The MFMA A operand V^T (d rows, kv slots) is read with
//            ds_read_b64_tr_b16 (four kv rows per read, so a half-wave touches
//            four rows whose 64-byte pieces the swizzle puts on different
//            banks); the kv rows of the two reads are chosen to match the slot
//            order of P^T: lane half g holds kv {4g..4g+3, 8+4g..8+4g+3} of
//            each 16-position group.
// KV rows past the end of the sequence are fetched from the last valid row (in
// bounds) and removed by the causal mask, which covers every such position.
// Cross-half exchanges (the two lanes that share a query column) use
// v_permlane32_swap instead of an LDS permute.
// ============================================================================
namespace fa2 {
constexpr int D = 128;
constexpr int BQ = 256;
constexpr int BKV = 64;
constexpr int NT = 512;
constexpr int NS = 5;                  // LDS ring stages (5 x 32 KB, all of LDS)
constexpr int SK = BKV * D / 8;        // u32x4 per K (or V) stage
constexpr int NL = 4;                  // DMA instructions per thread per stage
}  // namespace fa2

// Exchange between the wave halves: after the swap, a holds v of lanes
// 0..31 in both halves and b holds v of lanes 32..63 in both halves.  Written
// as inline asm because this compiler folds the builtin's two results into one
// when both inputs are the same value (r[0] + r[1] came out as r[0] + r[0]).
// The s_nop covers the VALU-write -> permlane-read hazard.
__device__ __forceinline__ void swap_halves(float& a, float& b) {
  asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
// max / sum of v over the two lanes l and l^32 (identical result in both).
__device__ __forceinline__ float xhalf_max(float v) {
  float a = v, b = v;
  swap_halves(a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float xhalf_sum(float v) {
  float a = v, b = v;
  swap_halves(a, b);
  return a + b;
}

template <int DT, int NS = fa2::NS>
__device__ __forceinline__ void prefill_tile_dma(const uint16_t* __restrict__ Q,
                                                 const uint16_t* __restrict__ K,
                                                 const uint16_t* __restrict__ V,
                                                 uint16_t* __restrict__ O, uint32_t seq_len,
                                                 uint32_t start_pos, uint32_t max_seq, uint32_t nh,
                                                 uint32_t nkv, float scale_log2, uint32_t bh,
                                                 uint32_t qb) {
  using fa2::BKV;
  using fa2::BQ;
  using fa2::D;
  using fa2::NL;
  using fa2::SK;
  using fa::kRescaleThreshold;
  static_assert(NS >= 4 && NS * 2 * SK * 16 <= 160 * 1024, "ring depth");
  u32x4* arena = lds::dma_lds_arena<NS * 2 * SK * 16>();
  auto lds_k = [&](int st) { return arena + st * 2 * SK; };
  auto lds_v = [&](int st) { return arena + st * 2 * SK + SK; };

  const uint32_t b = bh / nh, h = bh % nh;
  const uint32_t kvh = h / (nh / nkv);
  const uint32_t q0 = qb * BQ;
  const uint32_t kv_len = start_pos + seq_len;

  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int l32 = lane & 31, g = lane >> 5;
  const uint32_t qw0 = q0 + 32 * wave;
  const uint32_t my_q = qw0 + l32;
  const uint32_t qa_lo = start_pos + qw0;
  const uint32_t qa_hi = start_pos + qw0 + 31;
  const uint32_t my_qa = start_pos + my_q;

  const size_t q_row_stride = static_cast<size_t>(nh) * D;
  const uint16_t* kbase = K + (static_cast<size_t>(b) * nkv + kvh) * max_seq * D;
  const uint16_t* vbase = V + (static_cast<size_t>(b) * nkv + kvh) * max_seq * D;

  u32x4 qf[8];
  {
    const uint16_t* qp = Q + (static_cast<size_t>(b) * seq_len + my_q) * q_row_stride + h * D;
#pragma unroll
    for (int ds = 0; ds < 8; ++ds)
      qf[ds] = (my_q < seq_len) ? ldg128(qp + 16 * ds + 8 * g) : u32x4{0, 0, 0, 0};
  }

  const uint32_t q_hi_wg = min(q0 + BQ, seq_len);
  const uint32_t kv_need = start_pos + q_hi_wg;
  const uint32_t nkb = (kv_need + BKV - 1) / BKV;

  // ---- DMA: load j (0,1) of wave w fills 1 KB block 2w+j of the K and of the
  //      V stage; lane l owns 16-byte slot l of it (row = slot/16). ----
  int drow[2], kcol[2], vcol[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int slot = (2 * wave + j) * 64 + lane;
    const int row = slot >> 4, u = slot & 15;
    drow[j] = row;
    kcol[j] = 8 * (u ^ (row & 15));
    vcol[j] = 8 * (u ^ (4 * (row & 3)));
  }
  auto issue = [&](int st, uint32_t kb) {
    const uint32_t kv0 = kb * BKV;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const size_t pos = min(kv0 + drow[j], kv_len - 1);
      lds::dma16(kbase + pos * D + kcol[j], lds_k(st) + (2 * wave + j) * 64);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const size_t pos = min(kv0 + drow[j], kv_len - 1);
      lds::dma16(vbase + pos * D + vcol[j], lds_v(st) + (2 * wave + j) * 64);
    }
  };

  // V^T fragment (d tile dt, kv group st of 16) via two transposed reads.
  const int tq = lane >> 4, ti = lane & 15;
  auto read_v = [&](int stg, int st, int dt) {
    const char* vb = reinterpret_cast<const char*>(lds_v(stg));
    const int d = 32 * dt + 16 * (tq & 1) + 4 * (ti & 3);
    u32x4 f;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int kv = 16 * st + 4 * (tq >> 1) + 8 * r + (ti >> 2);
      const int off = kv * 256 + ((((d >> 3) ^ (4 * (kv & 3)))) << 4) + (d & 7) * 2;
      const u32x2 w = lds::read_tr16(vb + off);
      f[2 * r] = w[0];
      f[2 * r + 1] = w[1];
    }
    return f;
  };

  // This wave's KV blocks: [0, jd) lie wholly at or below the causal diagonal
  // of all its rows (and inside the sequence); [jd, ja) need the mask; blocks
  // from ja on are past every row's diagonal (or the wave has no rows).
  const uint32_t ja = (qw0 < seq_len) ? min(qa_hi / BKV + 1, nkb) : 0u;
  const uint32_t jd = min((qa_lo + 1) / BKV, ja);

  f32x16 o_acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) o_acc[i][r] = 0.0f;
  float m_run = -INFINITY;
  float l_run = 0.0f;

  // S^T = K.Q^T for the block in ring slot `stg` (raw scores).
  auto qk = [&](int stg, f32x16 (&acc)[2]) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][r] = 0.0f;
    const u32x4* kb = lds_k(stg);
#pragma unroll
    for (int ds = 0; ds < 8; ++ds) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const int row = 32 * kt + l32;
        const u32x4 kf = kb[row * 16 + ((2 * ds + g) ^ (row & 15))];
        acc[kt] = mfma32x32x16<DT>(kf, qf[ds], acc[kt]);
      }
    }
  };
  auto mask = [&](f32x16 (&sc)[2], uint32_t kv0) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const uint32_t pos = kv0 + 32 * kt + 8 * (r >> 2) + 4 * g + (r & 3);
        if (pos > my_qa) sc[kt][r] = -INFINITY;
      }
  };
  // Online-softmax step on the scores in sc (overwritten by P); branch-free.
  // The running max moves only when some row's block max exceeds it by more
  // than the threshold (exponents stay <= 2^threshold until then, which f32
  // sums and 16-bit P absorb).  hi = P as the 16-bit MFMA operand, per group
  // of 16 KV positions.  split: some key of this block carries more than
  // 1/kSplitRatio of its row's probability mass so far, so the rounding of
  // its P to 16 bits would show in O; then the residual P - hi(P) is
  // accumulated as well.
  auto softmax = [&](f32x16 (&sc)[2], u32x4 (&hi)[4], float& alpha, bool& grow, bool& split) {
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sc[kt][r]);
    mx = xhalf_max(mx);
    const float m_blk = mx * scale_log2;
    const bool growl = m_blk > m_run + kRescaleThreshold || m_run == -INFINITY;
    grow = __builtin_amdgcn_ballot_w64(growl) != 0;
    const float m_new = grow ? fmaxf(m_run, m_blk) : m_run;
    alpha = exp2_fast(m_run - m_new);
    m_run = m_new;
    // All exponentials first, then the row sum in two chains: an add that reads
    // the exp issued just before it waits a cycle (trans -> VALU hazard).
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) sc[kt][r] = exp2_fast(__builtin_fmaf(sc[kt][r], scale_log2, -m_new));
    float ls0 = 0.0f, ls1 = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      ls0 += sc[0][r];
      ls1 += sc[1][r];
    }
    l_run = __builtin_fmaf(l_run, alpha, ls0 + ls1);
    const float tot = xhalf_sum(l_run);
    const float pmax = exp2_fast(m_blk - m_new);
    split = __builtin_amdgcn_ballot_w64(pmax * fa::kSplitRatio<DT> > tot) != 0;
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int kt = st >> 1, hh = st & 1;
#pragma unroll
      for (int pp = 0; pp < 4; ++pp)
        hi[st][pp] = cvt_pk<DT>(sc[kt][8 * hh + 2 * pp], sc[kt][8 * hh + 2 * pp + 1]);
    }
  };
  // lo = P - hi(P) as 16-bit operands (only for split blocks).
  auto residual = [&](const f32x16 (&sc)[2], const u32x4 (&hi)[4], u32x4 (&lo)[4]) {
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int kt = st >> 1, hh = st & 1;
#pragma unroll
      for (int pp = 0; pp < 4; ++pp) {
        float a, c;
        unpack_pair<DT>(hi[st][pp], a, c);
        lo[st][pp] = cvt_pk<DT>(sc[kt][8 * hh + 2 * pp] - a, sc[kt][8 * hh + 2 * pp + 1] - c);
      }
    }
  };
  // O^T += V^T.P^T for the block in ring slot `stg`.
  auto pv = [&](int stg, const u32x4 (&hi)[4], const u32x4 (&lo)[4], bool split) {
#pragma unroll
    for (int st = 0; st < 4; ++st)
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
        o_acc[dt] = mfma32x32x16<DT>(read_v(stg, st, dt), hi[st], o_acc[dt]);
    if (split) {
#pragma unroll
      for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
          o_acc[dt] = mfma32x32x16<DT>(read_v(stg, st, dt), lo[st], o_acc[dt]);
    }
  };

  // Two wave groups share each SIMD (wave w and w+4).  Every wave runs the
  // same stream RA(0) RB(0) RA(1) RB(1) ..., where RA(j) = softmax of block j
  // fused with the QK MFMAs of block j+1 and RB(j) = the PV MFMAs of block j;
  // only the position of the per-block barrier differs: group A (waves 0-3)
  // meets it after RB(j), group B (waves 4-7) after RA(j).  Between two
  // barriers A therefore runs RA(j+1) RB(j+1) while B runs RB(j) RA(j+1): one
  // wave of each SIMD is in its VALU-heavy RA while the other is in its
  // MFMA-only RB.
  // Ring: between barriers j-1 and j the waves read K of block j+1 and V of
  // blocks j-1 (B) and j (A); block j+2 must have landed before barrier j,
  // and after it the slot of block j-1 is refilled with block j+NS-1.
  const bool grp_b = wave >= 4;
  u32x4 hi[4], lo[4];
  bool split = false;
  auto RA = [&](uint32_t j, f32x16 (&sc)[2], f32x16 (&sn)[2]) {
    if (j >= ja) return;
    const bool nxt = j + 1 < ja;
    const bool fused = j < jd && nxt;
    float alpha;
    bool grow;
    if (fused) {
      qk((j + 1) % NS, sn);
      softmax(sc, hi, alpha, grow, split);
    } else {
      if (j >= jd) mask(sc, j * BKV);
      softmax(sc, hi, alpha, grow, split);
    }
    if (grow) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) o_acc[i][r] *= alpha;
    }
    if (split) residual(sc, hi, lo);
  };
  auto RB = [&](uint32_t j, f32x16 (&sn)[2]) {
    if (j >= ja) return;
    pv(j % NS, hi, lo, split);
    if (!(j < jd && j + 1 < ja) && j + 1 < ja) qk((j + 1) % NS, sn);
  };
  auto sync = [&](uint32_t j) {
    if (j + 1 >= nkb) return;
    lds::wait_lgkm0();
    if (j + 2 < nkb) {
      if constexpr (NS >= 5)
        gemm::wait_stages<NL, NS - 4>(min(nkb - 3 - j, static_cast<uint32_t>(NS - 4)));
      else
        lds::wait_vm<0>();
    }
    lds::bar();
    if (j >= 1 && j + NS - 1 < nkb) issue((j - 1) % NS, j + NS - 1);
  };
  auto iteration = [&](uint32_t j, f32x16 (&sc)[2], f32x16 (&sn)[2]) {
    RA(j, sc, sn);
    if (grp_b) sync(j);
    RB(j, sn);
    if (!grp_b) sync(j);
  };

  // The previous work item of this workgroup (grid-stride callers) may still
  // be reading the ring.
  lds::bar();
#pragma unroll
  for (int s = 0; s < NS; ++s)
    if (static_cast<uint32_t>(s) < nkb) issue(s, s);
  gemm::wait_stages<NL, NS - 2>(nkb >= 2 ? min(nkb - 2, static_cast<uint32_t>(NS - 2)) : 0u);
  lds::bar();

  f32x16 sa[2], sb[2];
  if (ja > 0) qk(0, sa);
  for (uint32_t j = 0; j < nkb; j += 2) {
    iteration(j, sa, sb);
    if (j + 1 < nkb) iteration(j + 1, sb, sa);
  }

  const float l_tot = xhalf_sum(l_run);
  const float inv = 1.0f / l_tot;
  if (my_q < seq_len) {
    uint16_t* op = O + (static_cast<size_t>(b) * seq_len + my_q) * q_row_stride + h * D;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d = 32 * dt + 8 * q4 + 4 * g;
        u32x2 w;
        w[0] = cvt_pk<DT>(o_acc[dt][4 * q4 + 0] * inv, o_acc[dt][4 * q4 + 1] * inv);
        w[1] = cvt_pk<DT>(o_acc[dt][4 * q4 + 2] * inv, o_acc[dt][4 * q4 + 3] * inv);
        *reinterpret_cast<u32x2*>(op + d) = w;
      }
  }
}

template <int DT>
__global__ void __launch_bounds__(fa2::NT, 1)
attn_prefill_dma128(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
                    const uint16_t* __restrict__ V, uint16_t* __restrict__ O, uint32_t batch,
                    uint32_t seq_len, uint32_t start_pos, uint32_t max_seq, uint32_t nh,
                    uint32_t nkv, float scale_log2) {
  const uint32_t nqb = (seq_len + fa2::BQ - 1) / fa2::BQ;
  uint32_t bh, qb;
  prefill_work(blockIdx.x, batch * nh, nqb, bh, qb);
  prefill_tile_dma<DT>(Q, K, V, O, seq_len, start_pos, max_seq, nh, nkv, scale_log2, bh, qb);
}

// ============================================================================
// Decode: one query token per head, GQA group G = NH/NKV query heads share each
// K/V load.  Grid = B * NKV * n_split workgroups of 256 threads; each walks a
// run of consecutive 512-position chunks of one (batch, kv_head), per chunk:
//   A  scores S^T (16 kv x 16 q, G real columns) with v_mfma_f32_16x16x32, K
//      fragments read straight from HBM (each lane 4 x 16 B of one K row),
//   B  per-query max / exp / sum over the chunk (in LDS), merged into the
//      running (m, l) of the workgroup's run,
//   C  P.V on the vector ALUs in f32: each lane owns 8 d-values of every 4th row.
// With one split the workgroup writes O itself; otherwise each run's partial
// (m, l, O) goes to a workspace and attn_decode_combine merges them.
// K and V are read exactly once, with nontemporal loads (measured on MI355X:
// ~8% more sustained bandwidth than cached loads for this stream).
// ============================================================================
namespace dec {
constexpr int D = 128;
constexpr int CHUNK = 512;
constexpr int NT = 256;
constexpr int CT = 512;  // threads of the combine block
}  // namespace dec

// One work item: chunks [c_begin, c_end) of (batch, kv_head) `bk` = b*NKV + kvh.
// With `ws` non-null the chunk range's partial (m, l, O) goes to
// ws[((bk*G + q)*n_split + split)*(D+2)]; otherwise O = acc / l is written to
// `O` directly (the range must then cover the whole sequence).
// KP: phase A reads a wave's K rows in KP passes (fewer passes = more loads in
// flight per wave, more registers); VU: V rows in flight per wave in phase C.
template <int DT, int G, int KP = 4, int VU = 8>
__device__ __forceinline__ void decode_tile(const uint16_t* __restrict__ Q,
                                            const uint16_t* __restrict__ K,
                                            const uint16_t* __restrict__ V,
                                            uint16_t* __restrict__ O, float* __restrict__ ws,
                                            uint32_t seq_len, uint32_t max_seq, uint32_t nh,
                                            uint32_t nkv, uint32_t n_split, float scale_log2,
                                            uint32_t bk, uint32_t split, uint32_t c_begin,
                                            uint32_t c_end) {
  using namespace dec;
  __shared__ float sc[G][CHUNK];       // scores, then probabilities
  __shared__ float red[4][G][D];       // per-wave partial O
  __shared__ float stat_m[G], stat_l[G], stat_a[G];

  const uint32_t b = bk / nkv, kvh = bk % nkv;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int l16 = lane & 15, g4 = lane >> 4;

  u32x4 qf[4];
  {
    const uint32_t hq = kvh * G + l16;
    const uint16_t* qp = Q + (static_cast<size_t>(b) * nh + hq) * D;
#pragma unroll
    for (int s = 0; s < 4; ++s) qf[s] = (l16 < G) ? ldg128(qp + 32 * s + 8 * g4) : u32x4{0, 0, 0, 0};
  }
  if (t < G) {
    stat_m[t] = -INFINITY;
    stat_l[t] = 0.0f;
  }

  float acc[G][8];
#pragma unroll
  for (int q = 0; q < G; ++q)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[q][e] = 0.0f;
  const int dc = l16;  // this lane's d range in phase C: 8*dc .. 8*dc+7

  for (uint32_t ch = c_begin; ch < c_end; ++ch) {
    const uint32_t c0 = ch * CHUNK;
    const uint32_t n_here = (c0 < seq_len) ? min(static_cast<uint32_t>(CHUNK), seq_len - c0) : 0u;
    const uint16_t* kb = K + (static_cast<size_t>(bk) * max_seq + c0) * D;
    const uint16_t* vb = V + (static_cast<size_t>(bk) * max_seq + c0) * D;

    // ---- phase A: scores S^T = K . Q^T, 16 rows per MFMA tile ----
    {
      constexpr int TILES = CHUNK / 4 / 16;  // per wave
      constexpr int TP = TILES / KP;          // tiles whose K rows are in flight together
      static_assert(TILES % KP == 0, "K passes");
#pragma unroll
      for (int half = 0; half < KP; ++half) {
        u32x4 kf[TP][4];
#pragma unroll
        for (int tt = 0; tt < TP; ++tt) {
          const uint32_t row = wave * (CHUNK / 4) + (half * TP + tt) * 16 + l16;
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const uint16_t* kp = kb + static_cast<size_t>(row) * D + 32 * s + 8 * g4;
            kf[tt][s] = (row < n_here) ? ldg128_nt(kp) : u32x4{0, 0, 0, 0};
          }
        }
#pragma unroll
        for (int tt = 0; tt < TP; ++tt) {
          f32x4 a4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int s = 0; s < 4; ++s) a4 = mfma16x16x32<DT>(kf[tt][s], qf[s], a4);
          const uint32_t row0 = wave * (CHUNK / 4) + (half * TP + tt) * 16 + 4 * g4;
          if (l16 < G) {
            f32x4 w;
#pragma unroll
            for (int i = 0; i < 4; ++i) w[i] = (row0 + i < n_here) ? a4[i] * scale_log2 : -INFINITY;
            *reinterpret_cast<f32x4*>(&sc[l16][row0]) = w;
          }
        }
      }
    }
    __syncthreads();

    // ---- phase B: per-query max, exp, sum; merge with the running (m, l) ----
    for (int q = wave; q < G; q += 4) {
      float mx = -INFINITY;
      for (int i = lane; i < CHUNK; i += 64) mx = fmaxf(mx, sc[q][i]);
      mx = wave_max(mx);
      const float m_old = stat_m[q];
      const float m_new = fmaxf(m_old, mx);
      float sum = 0.0f;
      for (int i = lane; i < CHUNK; i += 64) {
        const float p = (m_new == -INFINITY) ? 0.0f : exp2_fast(sc[q][i] - m_new);
        sc[q][i] = p;
        sum += p;
      }
      sum = wave_sum(sum);
      if (lane == 0) {
        const float alpha = (m_old == -INFINITY) ? 0.0f : exp2_fast(m_old - m_new);
        stat_a[q] = alpha;
        stat_l[q] = stat_l[q] * alpha + sum;
        stat_m[q] = m_new;
      }
    }
    __syncthreads();

    // ---- phase C: acc = acc * alpha + sum_pos p[q][pos] * V[pos][d] ----
    {
#pragma unroll
      for (int q = 0; q < G; ++q) {
        const float a = stat_a[q];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[q][e] *= a;
      }
      constexpr int ROWS_PER_WAVE = CHUNK / 4;
      constexpr int UNROLL = VU;
      static_assert((ROWS_PER_WAVE / 4) % UNROLL == 0, "V rows per pass");
#pragma unroll 1
      for (int it = 0; it < ROWS_PER_WAVE / 4; it += UNROLL) {
        u32x4 vv[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
          const uint32_t row = wave * ROWS_PER_WAVE + 4 * (it + u) + g4;
          const uint16_t* vp = vb + static_cast<size_t>(row) * D + 8 * dc;
          vv[u] = (row < n_here) ? ldg128_nt(vp) : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
          const int row = wave * ROWS_PER_WAVE + 4 * (it + u) + g4;
          float vf[8];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            vf[2 * e] = u16_to_f32<DT>(static_cast<uint16_t>(vv[u][e] & 0xffffu));
            vf[2 * e + 1] = u16_to_f32<DT>(static_cast<uint16_t>(vv[u][e] >> 16));
          }
#pragma unroll
          for (int q = 0; q < G; ++q) {
            const float p = sc[q][row];
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[q][e] = __builtin_fmaf(p, vf[e], acc[q][e]);
          }
        }
      }
    }
    __syncthreads();  // sc and stat_a are rewritten by the next chunk
  }

  // reduce the 4 row groups of each wave (lanes l, l^16, l^32, l^48), then the waves
#pragma unroll
  for (int q = 0; q < G; ++q)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = acc[q][e];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      acc[q][e] = v;
    }
  if (g4 == 0) {
#pragma unroll
    for (int q = 0; q < G; ++q)
#pragma unroll
      for (int e = 0; e < 8; ++e) red[wave][q][8 * dc + e] = acc[q][e];
  }
  __syncthreads();

  for (int i = t; i < G * D; i += NT) {
    const int q = i / D, d = i % D;
    const float o = red[0][q][d] + red[1][q][d] + red[2][q][d] + red[3][q][d];
    if (ws) {
      float* rec = ws + ((static_cast<size_t>(bk) * G + q) * n_split + split) * (D + 2);
      rec[2 + d] = o;
      if (d == 0) {
        rec[0] = stat_m[q];
        rec[1] = stat_l[q];
      }
    } else {
      const float l = stat_l[q];
      const float v = (l > 0.0f) ? o / l : 0.0f;
      O[(static_cast<size_t>(b) * nh + kvh * G + q) * D + d] = f32_to_u16<DT>(v);
    }
  }
  __syncthreads();  // red and stat_* are reused by the next work item
}

// Library path: n_split workgroups per (batch, kv_head), each walking `cps`
// consecutive chunks (the host picks both so that every split has at least one
// chunk).  With n_split == 1 a workgroup covers the whole sequence and writes O;
// otherwise its partial goes to the workspace for attn_decode_combine.
template <int DT, int G>
__global__ void __launch_bounds__(dec::NT)
attn_decode_split(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
                  const uint16_t* __restrict__ V, uint16_t* __restrict__ O, float* __restrict__ ws,
                  uint32_t seq_len, uint32_t max_seq, uint32_t nh, uint32_t nkv, uint32_t n_split,
                  uint32_t cps, float scale_log2) {
  const uint32_t nchunks = (seq_len + dec::CHUNK - 1) / dec::CHUNK;
  const uint32_t split = blockIdx.x % n_split;
  const uint32_t bk = blockIdx.x / n_split;
  const uint32_t c0 = split * cps, c1 = min(nchunks, c0 + cps);
  decode_tile<DT, G>(Q, K, V, O, n_split > 1 ? ws : nullptr, seq_len, max_seq, nh, nkv, n_split,
                     scale_log2, bk, split, c0, c1);
}

// Merge the per-chunk partials: O = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s.
// One 512-thread block per (batch, head).  The chunk statistics (m_s, l_s) come
// in with one load per thread per 512 chunks and M is reduced over the block.
// Then four groups of 128 threads (thread d of a group owns output d) each merge
// a contiguous quarter of the chunks with sixteen O loads in flight, and the
// four partial sums are added in group order.  The merge is latency-bound (a
// few KB per head), so it is built to need few memory round trips: statistics,
// then ceil(n_split / 64) rounds of O loads.
template <int DT>
__global__ void __launch_bounds__(dec::CT)
attn_decode_combine(const float* __restrict__ ws, uint16_t* __restrict__ O, uint32_t nh,
                    uint32_t nkv, uint32_t n_split) {
  constexpr int D = dec::D, CT = dec::CT, NG = CT / D, UNR = 16;
  __shared__ float s_w[CT], s_l[CT];
  __shared__ float s_max[CT / 64];
  __shared__ float s_num[NG][D], s_den[NG][D];
  const uint32_t bhq = blockIdx.x;  // b * nh + h
  const uint32_t b = bhq / nh, h = bhq % nh;
  const uint32_t G = nh / nkv;
  const uint32_t kvh = h / G, q = h % G;
  const float* rec0 = ws + ((static_cast<size_t>(b) * nkv + kvh) * G + q) * n_split * (D + 2);
  const int t = threadIdx.x, d = t % D, grp = t / D;

  // M = max_s m_s; the first pass's (m, l) stay in registers.
  float m_own = -INFINITY, l_own = 0.0f, mx = -INFINITY;
  for (uint32_t s0 = 0; s0 < n_split; s0 += CT) {
    if (s0 + t < n_split) {
      const float m = rec0[(s0 + t) * (D + 2)];
      if (s0 == 0) {
        m_own = m;
        l_own = rec0[t * (D + 2) + 1];
      }
      mx = fmaxf(mx, m);
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if ((t & 63) == 0) s_max[t >> 6] = mx;
  __syncthreads();
  float M = s_max[0];
#pragma unroll
  for (int w = 1; w < CT / 64; ++w) M = fmaxf(M, s_max[w]);

  float num = 0.0f, den = 0.0f;
  for (uint32_t s0 = 0; s0 < n_split; s0 += CT) {
    const uint32_t cnt = min(static_cast<uint32_t>(CT), n_split - s0);
    if (s0 > 0) __syncthreads();  // the previous pass is done with s_w / s_l
    if (static_cast<uint32_t>(t) < cnt) {
      float m = m_own, l = l_own;
      if (s0 > 0) {
        const float* rec = rec0 + (s0 + t) * (D + 2);
        m = rec[0];
        l = rec[1];
      }
      s_w[t] = (m == -INFINITY) ? 0.0f : exp2_fast(m - M);
      s_l[t] = l;
    }
    __syncthreads();
    const uint32_t per = (cnt + NG - 1) / NG;
    const uint32_t lo = min(cnt, grp * per), hi = min(cnt, lo + per);
    const float* od = rec0 + static_cast<size_t>(s0) * (D + 2) + 2 + d;
    uint32_t i = lo;
    for (; i + UNR <= hi; i += UNR) {
      float o[UNR];
#pragma unroll
      for (int u = 0; u < UNR; ++u) o[u] = od[(i + u) * (D + 2)];
#pragma unroll
      for (int u = 0; u < UNR; ++u) {
        num = __builtin_fmaf(s_w[i + u], o[u], num);
        den = __builtin_fmaf(s_w[i + u], s_l[i + u], den);
      }
    }
    for (; i < hi; ++i) {
      num = __builtin_fmaf(s_w[i], od[i * (D + 2)], num);
      den = __builtin_fmaf(s_w[i], s_l[i], den);
    }
  }
  s_num[grp][d] = num;
  s_den[grp][d] = den;
  __syncthreads();
  if (grp == 0) {
    float n = s_num[0][d], dd = s_den[0][d];
#pragma unroll
    for (int g = 1; g < NG; ++g) {
      n += s_num[g][d];
      dd += s_den[g][d];
    }
    const float o = (dd > 0.0f) ? n / dd : 0.0f;
    O[static_cast<size_t>(bhq) * D + d] = f32_to_u16<DT>(o);
  }
}

// ============================================================================
// General attention: any head_dim <= 256, any dtype (f32 / f16 / bf16), causal
// or not.  One 256-thread workgroup per (batch, query, head); KV streamed in
// chunks of 1024 scores kept in LDS, online softmax across chunks.  Used for
// shapes outside the fast kernels and for the f32 single-head op.
//   kv_visible(q) = causal ? min(start_pos + q + 1, kv_len) : kv_len
// q_pos_stride is the element stride between consecutive query rows of one head
// (NH*D for [S][NH][D]); kv tensors are [B][NKV][max_seq][D].
// ============================================================================
namespace gen_attn {
constexpr int CH = 1024;   // scores per pass
template <int NT>
constexpr int smem_floats() { return 256 + CH + NT / 64; }
}  // namespace gen_attn

// `smem` (LDS, gen_attn::smem_floats<NT>() floats) holds the query row, one pass of
// scores and the cross-wave reduction slots; a kernel that also runs an
// LDS-filling path passes part of that path's arena.
template <int DT, int NT = 256>
__device__ __forceinline__ void attn_general_item_smem(
    const void* __restrict__ Q, const void* __restrict__ K, const void* __restrict__ V,
    void* __restrict__ O, uint32_t seq_len, uint32_t start_pos, uint32_t max_seq,
    uint32_t kv_len, uint32_t head_dim, uint32_t nh, uint32_t nkv, int causal, float scale,
    uint32_t item, float* smem) {
  constexpr int CH = gen_attn::CH;
  constexpr int NW = NT / 64;
  static_assert(NT >= 256 && NT % 64 == 0, "head_dim up to 256 needs >= 256 threads");
  float* qs = smem;
  float* sc = smem + 256;
  float* red = smem + 256 + CH;
  const uint32_t h = item % nh;
  const uint32_t qi = (item / nh) % seq_len;
  const uint32_t b = item / (nh * seq_len);
  const uint32_t kvh = h / (nh / nkv);
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  auto ld = [&](const void* p, size_t i) -> float {
    if constexpr (DT == kF32) return static_cast<const float*>(p)[i];
    else return u16_to_f32<DT>(static_cast<const uint16_t*>(p)[i]);
  };
  const size_t q_off = ((static_cast<size_t>(b) * seq_len + qi) * nh + h) * head_dim;
  const size_t kv_off = (static_cast<size_t>(b) * nkv + kvh) * max_seq * head_dim;
  for (uint32_t d = t; d < head_dim; d += NT) qs[d] = ld(Q, q_off + d);
  __syncthreads();
  const uint32_t visible = causal ? min(start_pos + qi + 1, kv_len) : kv_len;
  float m_run = -INFINITY, l_run = 0.0f, acc = 0.0f;  // acc: d = t
  for (uint32_t c0 = 0; c0 < visible; c0 += CH) {
    const uint32_t n = min(static_cast<uint32_t>(CH), visible - c0);
    for (uint32_t p = t; p < n; p += NT) {
      const size_t kr = kv_off + static_cast<size_t>(c0 + p) * head_dim;
      float dot = 0.0f;
      for (uint32_t d = 0; d < head_dim; ++d) dot = __builtin_fmaf(qs[d], ld(K, kr + d), dot);
      sc[p] = dot * scale;
    }
    __syncthreads();
    float mx = -INFINITY;
    for (uint32_t p = t; p < n; p += NT) mx = fmaxf(mx, sc[p]);
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) mx = fmaxf(mx, red[w]);
    __syncthreads();
    const float m_new = fmaxf(m_run, mx);
    const float alpha = expf(m_run - m_new);
    float sum = 0.0f;
    for (uint32_t p = t; p < n; p += NT) {
      const float e = expf(sc[p] - m_new);
      sc[p] = e;
      sum += e;
    }
    sum = wave_sum(sum);
    if (lane == 0) red[wave] = sum;
    __syncthreads();
    sum = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) sum += red[w];
    l_run = l_run * alpha + sum;
    if (static_cast<uint32_t>(t) < head_dim) {
      float a = acc * alpha;
      for (uint32_t p = 0; p < n; ++p)
        a = __builtin_fmaf(sc[p], ld(V, kv_off + static_cast<size_t>(c0 + p) * head_dim + t), a);
      acc = a;
    }
    m_run = m_new;
    __syncthreads();
  }
  if (static_cast<uint32_t>(t) < head_dim) {
    const float o = (l_run > 0.0f) ? acc / l_run : 0.0f;
    if constexpr (DT == kF32) static_cast<float*>(O)[q_off + t] = o;
    else static_cast<uint16_t*>(O)[q_off + t] = f32_to_u16<DT>(o);
  }
  __syncthreads();  // smem is reused by the next item
}

template <int DT, int NT = 256>
__device__ __forceinline__ void attn_general_item(
    const void* __restrict__ Q, const void* __restrict__ K, const void* __restrict__ V,
    void* __restrict__ O, uint32_t seq_len, uint32_t start_pos, uint32_t max_seq,
    uint32_t kv_len, uint32_t head_dim, uint32_t nh, uint32_t nkv, int causal, float scale,
    uint32_t item) {
  __shared__ float smem[gen_attn::smem_floats<NT>()];
  attn_general_item_smem<DT, NT>(Q, K, V, O, seq_len, start_pos, max_seq, kv_len, head_dim, nh,
                                 nkv, causal, scale, item, smem);
}

template <int DT>
__global__ void __launch_bounds__(256)
attn_general(const void* __restrict__ Q, const void* __restrict__ K, const void* __restrict__ V,
             void* __restrict__ O, uint32_t batch, uint32_t seq_len, uint32_t start_pos,
             uint32_t max_seq, uint32_t kv_len, uint32_t head_dim, uint32_t nh, uint32_t nkv,
             int causal, float scale) {
  (void)batch;
  attn_general_item<DT>(Q, K, V, O, seq_len, start_pos, max_seq, kv_len, head_dim, nh, nkv,
                        causal, scale, blockIdx.x);
}

// Causal mask on an f32 tile (mlir_to_linalg.rs:1191-1247): y = x where col <= row,
// else -inf.  Bit-exact.  Rows are `rows` long tiles stacked `tiles` deep.
__global__ void __launch_bounds__(256)
causal_mask_f32(const float* __restrict__ x, float* __restrict__ y, uint32_t rows, uint32_t cols,
                uint64_t total) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= total) return;
  const uint32_t c = static_cast<uint32_t>(i % cols);
  const uint32_t r = static_cast<uint32_t>((i / cols) % rows);
  y[i] = (c <= r) ? x[i] : __uint_as_float(0xff800000u);
}

}  // namespace th
