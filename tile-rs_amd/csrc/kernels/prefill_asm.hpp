// Causal GQA prefill, head_dim 128, 16-bit Q/K/V: the library's kernel.
//
// The main loop is generated gfx950 assembly (gen_prefill.py, run by the build
// into kernels/gen/prefill_asm.inc); this wrapper computes the per-lane and
// per-wave operands and hands everything to one asm statement, which loads Q,
// streams K/V through the LDS ring, and writes O.  Work split, arithmetic and LDS
// layouts are described in gen_prefill.py.  Semantics: causal softmax(Q.K^T *
// rsqrt(D)).V over kv positions <= start_pos + row
// (/root/reference/crates/rustc_codegen_tile/src/mlir_to_msl.rs:10928-11009).
#pragma once
#include "attention.hpp"
#include "kernels/gen/prefill_asm.inc"

namespace th {
namespace pfa {
constexpr int D = 128;
constexpr int BQ = 256;   // query rows per workgroup
constexpr int BKV = 64;   // kv positions per ring stage
constexpr int NT = 512;   // 8 waves x 32 query rows
constexpr int NS = 5;     // ring stages (5 x 32 KB = all of LDS)

// Split-KV parts (PART): the workgroup covers K/V blocks [j0, j1) of its query block
// (j1 = ~0u: through the last) and writes, per query row, the unnormalized O in f32
// plus the row's sum l and running max m (log2 units) to part_out: a record of
// part_rec(HD) floats {O[HD], l, m, pad, pad} at row index q_row.  j0 * 64 must not
// exceed start_pos, so that every row of the part has an unmasked position (finite m).
__host__ __device__ constexpr int part_rec(int hd) { return hd + 4; }

// HD: head dim, 128 or 64.  Both use the same 160 KB LDS allocation (a kernel that
// instantiates both keeps one); at 64 the 5-stage ring fills half of it.  K stage
// [HD/128 halves][64 rows][8 chunks] x 16 B, chunk c of row r at c ^ kswz(r) (below; HD
// 64: one half); V stage row-major with 16-byte chunk c
// of row r at c ^ 4(r & 3) (HD 128) or c ^ 4((r >> 1) & 1) (HD 64): the four rows a
// transposed read touches then fall in distinct banks.
template <int DT, bool PART = false, int HD = D>
__device__ __forceinline__ void prefill_tile(const uint16_t* __restrict__ Q,
                                             const uint16_t* __restrict__ K,
                                             const uint16_t* __restrict__ V,
                                             uint16_t* __restrict__ O, uint32_t seq_len,
                                             uint32_t start_pos, uint32_t max_seq, uint32_t nh,
                                             uint32_t nkv, float scale_log2, uint32_t bh,
                                             uint32_t qb, bool head_major = false,
                                             uint32_t j0 = 0, uint32_t j1 = ~0u,
                                             float* __restrict__ part_out = nullptr) {
  static_assert(HD == 128 || HD == 64, "prefill head dim");
  constexpr uint32_t RB = 2 * HD;           // bytes of a K/V row
  u32x4* arena = lds::dma_lds_arena<NS * 2 * BKV * D * 2>();
  typedef __attribute__((address_space(3))) const void* lds_cptr;
  const uint32_t lds_base =
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_cptr)(arena)));

  const uint32_t b = bh / nh, h = bh % nh;
  const uint32_t kvh = h / (nh / nkv);
  const uint32_t q0 = qb * BQ;
  const uint32_t kv_len = start_pos + seq_len;
  const int lane = threadIdx.x & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l32 = lane & 31, g = lane >> 5;

  // Rows past seq_len are computed on the last row's data and not stored.  Q and O
  // are [B][S][NH][D], or [B][NH][S][D] with head_major.
  const uint32_t qt = q0 + 32 * wave + l32;
  const uint32_t qc = min(qt, seq_len - 1);
  const size_t q_row = head_major ? (static_cast<size_t>(b) * nh + h) * seq_len + qc
                                  : (static_cast<size_t>(b) * seq_len + qc) * nh + h;
  const uint16_t* qp = Q + q_row * HD + 8 * g;
  void* op = PART ? static_cast<void*>(part_out + q_row * part_rec(HD) + 4 * g)
                 : static_cast<void*>(O + q_row * HD + 4 * g);
  const uint64_t ok = __builtin_amdgcn_ballot_w64(qt < seq_len);
  // score (kt, r) of lane is kv position kv0 + 32kt + 8(r/4) + r%4 + 4g: masked
  // when that offset exceeds lim - kv0
  // The loop sees blocks j0 .. j1-1 as 0 .. nb-1: positions, the mask limit and the
  // block indices below are taken relative to position 64 * j0.
  const uint32_t q_hi_wg = min(q0 + BQ, seq_len);
  const uint32_t nb_all = (start_pos + q_hi_wg + BKV - 1) / BKV;
  const uint32_t jend = min(j1, nb_all);
  const uint32_t nb = jend - j0;
  const uint32_t p0 = j0 * BKV;
  const int lim = static_cast<int>(start_pos + qt - p0) - 4 * g;

  const uint64_t kbase = reinterpret_cast<uint64_t>(K + ((static_cast<size_t>(b) * nkv + kvh) * max_seq + p0) * HD);
  const uint64_t vbase = reinterpret_cast<uint64_t>(V + ((static_cast<size_t>(b) * nkv + kvh) * max_seq + p0) * HD);
  // DMA rows are clamped here (in bounds; masked or past the part)
  const uint32_t kvlast = min(kv_len, jend * BKV) - 1 - p0;
  const uint32_t jd = __builtin_amdgcn_readfirstlane((start_pos + q0 + 32 * wave + 1) / BKV - j0);
  // the wave's last kv block with an unmasked score (row q0 + 32 wave + 31)
  const uint32_t jl = __builtin_amdgcn_readfirstlane((start_pos + q0 + 32 * wave + 31) / BKV - j0);

  // LDS read offsets: K fragment rows (l32) and chunk g; V^T transposed reads
  auto vswz = [](uint32_t r) { return HD == 128 ? 4 * (r & 3) : 4 * ((r >> 1) & 1); };
  // K fragment (32 rows x 16 B): lane reads row l32, chunk 2 ds + g (the program XORs
  // 32 (ds & 3) and adds the row block and half as immediates).  The chunk swizzle
  // kswz(r) takes rows 1-2 and 4: a ds_read_b128 conflict window pairs lanes l .. l+7
  // with l+16 .. l+23 (rows r and r + 16), which then fall in distinct banks (with
  // r & 7 instead: 32% of LDS-active cycles in bank conflicts, measured).
  auto kswz = [](uint32_t r) { return ((r >> 1) & 3u) | ((r >> 2) & 4u); };
  const uint32_t klane = 128u * l32 + 16u * (static_cast<uint32_t>(g) ^ kswz(l32));
  uint32_t vlane;
  {
    const uint32_t d = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    const uint32_t kv = 4 * ((lane >> 4) >> 1) + ((lane & 15) >> 2);
    vlane = kv * RB + (((d >> 3) ^ vswz(kv)) << 4) + (d & 7) * 2;
  }
  // DMA in 1 KB units (HD/64 of K and as many of V per wave and block).  K unit u
  // holds half u / 8, rows 8 (u % 8) + lane / 8, chunk (lane % 8) ^ kswz(row) of the
  // half (whole 128-byte lines; unit j = 1 is 8 rows on, same kswz); HD 128: units
  // 2 wave + j, HD 64: unit wave.  V unit bi
  // holds row 4 bi + lane/16, chunk lane%16 ^ swizzle (HD 128), or row 8 wave + lane/8,
  // chunk lane%8 ^ swizzle (HD 64).
  const uint32_t krow = (HD == 128 ? 16 * (wave & 3) : 8 * wave) + (lane >> 3);
  const uint32_t kcol = (HD == 128 ? 128 * (wave >> 2) : 0) + 16 * ((lane & 7) ^ kswz(krow));
  const uint32_t vrow = HD == 128 ? 8 * wave + (lane >> 4) : 8 * wave + (lane >> 3);
  const uint32_t vcol = HD == 128 ? 16 * ((lane & 15) ^ vswz(vrow)) : 16 * ((lane & 7) ^ vswz(vrow));
  const uint32_t wave2k = (HD == 128 ? 2048 : 1024) * wave;
  // log2 of the residual-split ratio (a power of two, so exact)
  const float lratio = __builtin_log2f(fa::kSplitRatio<DT>);

#define TH_PREFILL_OPS(STR)                                                                \
  asm volatile(STR                                                                         \
               :                                                                           \
               : "v"(qp), "v"(op), "v"(lim), "v"(klane), "v"(vlane), "v"(krow), "v"(kcol), \
                 "v"(vrow), "v"(vcol), "s"(kbase), "s"(vbase), "s"(kvlast), "s"(nb),       \
                 "s"(jd), "s"(lds_base), "s"(wave2k), "s"(scale_log2), "s"(lratio), "s"(ok), \
                 "s"(jl)                                                                   \
               : TH_PREFILL_ASM_CLOBBERS, "vcc", "scc", "memory")
  if constexpr (HD == 64) {
    if constexpr (PART) {
      if constexpr (DT == kBF16) TH_PREFILL_OPS(TH_PREFILL_ASM_BF16_PART_D64); else TH_PREFILL_OPS(TH_PREFILL_ASM_F16_PART_D64);
    } else {
      if constexpr (DT == kBF16) TH_PREFILL_OPS(TH_PREFILL_ASM_BF16_D64); else TH_PREFILL_OPS(TH_PREFILL_ASM_F16_D64);
    }
  } else if constexpr (PART) {
    if constexpr (DT == kBF16) TH_PREFILL_OPS(TH_PREFILL_ASM_BF16_PART); else TH_PREFILL_OPS(TH_PREFILL_ASM_F16_PART);
  } else {
    if constexpr (DT == kBF16) TH_PREFILL_OPS(TH_PREFILL_ASM_BF16); else TH_PREFILL_OPS(TH_PREFILL_ASM_F16);
  }
#undef TH_PREFILL_OPS
}

// Grid = ceil(seq_len/256) * batch * num_heads workgroups of 512 threads, heavy
// (late) query blocks first.
template <int DT, int HD = D>
__global__ void __launch_bounds__(NT, 1)
attn_prefill_asm(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
                 const uint16_t* __restrict__ V, uint16_t* __restrict__ O, uint32_t batch,
                 uint32_t seq_len, uint32_t start_pos, uint32_t max_seq, uint32_t nh,
                 uint32_t nkv, float scale_log2) {
  const uint32_t nqb = (seq_len + BQ - 1) / BQ;
  uint32_t bh, qb;
  prefill_work(blockIdx.x, batch, nh, nkv, nqb, bh, qb);
  prefill_tile<DT, false, HD>(Q, K, V, O, seq_len, start_pos, max_seq, nh, nkv, scale_log2, bh, qb);
}
// Split-KV prefill for launches with fewer work items than CUs (chunked prefill after a
// long cache).  Workgroup w = item * nsplit + part; part p < nsplit-1 covers blocks
// [p c, (p+1) c), the last one [(nsplit-1) c, end), with c * (nsplit - 1) * 64 <=
// start_pos (checked on the host).  Partials go to ws: [nsplit][rows][part_rec(HD)] f32.
template <int DT, int HD = D>
__global__ void __launch_bounds__(NT, 1)
attn_prefill_split(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
                   const uint16_t* __restrict__ V, float* __restrict__ ws, uint32_t batch,
                   uint32_t seq_len, uint32_t start_pos, uint32_t max_seq, uint32_t nh,
                   uint32_t nkv, float scale_log2, uint32_t nsplit, uint32_t chunk) {
  const uint32_t nqb = (seq_len + BQ - 1) / BQ;
  const uint32_t item = blockIdx.x / nsplit, part = blockIdx.x % nsplit;
  uint32_t bh, qb;
  prefill_work(item, batch, nh, nkv, nqb, bh, qb);
  const size_t rows = static_cast<size_t>(batch) * seq_len * nh;
  const uint32_t j0 = part * chunk, j1 = part + 1 == nsplit ? ~0u : j0 + chunk;
  prefill_tile<DT, true, HD>(Q, K, V, nullptr, seq_len, start_pos, max_seq, nh, nkv, scale_log2,
                             bh, qb, false, j0, j1, ws + part * rows * part_rec(HD));
}

// Merge the split parts of each query row: O = sum_p 2^(m_p - M) O_p / sum_p 2^(m_p - M) l_p
// with M = max_p m_p.  HD/4 threads per row, four O values each; 256 threads per
// workgroup (8 rows at HD 128, 16 at 64).
template <int DT, int HD = D>
__global__ void __launch_bounds__(256)
attn_prefill_combine(const float* __restrict__ ws, uint16_t* __restrict__ O, size_t rows,
                     uint32_t nsplit) {
  constexpr int TPR = HD / 4, RPB = 256 / TPR, R = part_rec(HD);
  const size_t row = static_cast<size_t>(blockIdx.x) * RPB + threadIdx.x / TPR;
  if (row >= rows) return;
  const int c = threadIdx.x % TPR;
  const size_t pstride = rows * R;
  const float* rec = ws + row * R;
  float M = -INFINITY;
  for (uint32_t p = 0; p < nsplit; ++p) M = fmaxf(M, rec[p * pstride + HD + 1]);
  float den = 0.0f, num[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (uint32_t p = 0; p < nsplit; ++p) {
    const float* r = rec + p * pstride;
    const float w = exp2f(r[HD + 1] - M);
    den = __builtin_fmaf(w, r[HD], den);
    const float4 o = *reinterpret_cast<const float4*>(r + 4 * c);
    num[0] = __builtin_fmaf(w, o.x, num[0]);
    num[1] = __builtin_fmaf(w, o.y, num[1]);
    num[2] = __builtin_fmaf(w, o.z, num[2]);
    num[3] = __builtin_fmaf(w, o.w, num[3]);
  }
  const float inv = 1.0f / den;
  u32x2 out;
  out[0] = static_cast<uint32_t>(f32_to_u16<DT>(num[0] * inv)) |
           (static_cast<uint32_t>(f32_to_u16<DT>(num[1] * inv)) << 16);
  out[1] = static_cast<uint32_t>(f32_to_u16<DT>(num[2] * inv)) |
           (static_cast<uint32_t>(f32_to_u16<DT>(num[3] * inv)) << 16);
  *reinterpret_cast<u32x2*>(O + row * HD + 4 * c) = out;
}
}  // namespace pfa
}  // namespace th
