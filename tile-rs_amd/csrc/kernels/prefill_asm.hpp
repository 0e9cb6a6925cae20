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

template <int DT>
__device__ __forceinline__ void prefill_tile(const uint16_t* __restrict__ Q,
                                             const uint16_t* __restrict__ K,
                                             const uint16_t* __restrict__ V,
                                             uint16_t* __restrict__ O, uint32_t seq_len,
                                             uint32_t start_pos, uint32_t max_seq, uint32_t nh,
                                             uint32_t nkv, float scale_log2, uint32_t bh,
                                             uint32_t qb, bool head_major = false) {
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
  const uint16_t* qp = Q + q_row * D + 8 * g;
  uint16_t* op = O + q_row * D + 4 * g;
  const uint64_t ok = __builtin_amdgcn_ballot_w64(qt < seq_len);
  // score (kt, r) of lane is kv position kv0 + 32kt + 8(r/4) + r%4 + 4g: masked
  // when that offset exceeds lim - kv0
  const int lim = static_cast<int>(start_pos + qt) - 4 * g;

  const uint64_t kbase = reinterpret_cast<uint64_t>(K + (static_cast<size_t>(b) * nkv + kvh) * max_seq * D);
  const uint64_t vbase = reinterpret_cast<uint64_t>(V + (static_cast<size_t>(b) * nkv + kvh) * max_seq * D);
  const uint32_t kvlast = kv_len - 1;   // DMA rows are clamped here (in bounds; masked)
  const uint32_t q_hi_wg = min(q0 + BQ, seq_len);
  const uint32_t nb = (start_pos + q_hi_wg + BKV - 1) / BKV;
  const uint32_t jd = __builtin_amdgcn_readfirstlane((start_pos + q0 + 32 * wave + 1) / BKV);
  // the wave's last kv block with an unmasked score (row q0 + 32 wave + 31)
  const uint32_t jl = __builtin_amdgcn_readfirstlane((start_pos + q0 + 32 * wave + 31) / BKV);

  // LDS read offsets: K fragment rows (l32) and chunk g; V^T transposed reads
  const uint32_t klane = 16u * (256u * (l32 >> 4) + 16u * g + (l32 & 15));
  uint32_t vlane;
  {
    const int d = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    const int kv = 4 * ((lane >> 4) >> 1) + ((lane & 15) >> 2);
    vlane = kv * 256 + (((d >> 3) ^ (4 * (kv & 3))) << 4) + (d & 7) * 2;
  }
  // DMA: 1 KB unit bi = 2 wave + j of a stage; K unit bi holds rows
  // 16(bi/4) + lane%16, chunk 4(bi%4) + lane/16; V unit bi holds row
  // 4 bi + lane/16 with chunk lane%16 ^ 4(row%4)
  const uint32_t krow = 16 * (wave >> 1) + (lane & 15);
  const uint32_t kcol = 128 * (wave & 1) + 16 * (lane >> 4);
  const uint32_t vrow = 8 * wave + (lane >> 4);
  const uint32_t vcol = 16 * ((lane & 15) ^ (4 * (lane >> 4)));
  const uint32_t wave2k = 2048 * wave;
  // log2 of the residual-split ratio (a power of two, so exact)
  const float lratio = __builtin_log2f(fa::kSplitRatio<DT>);

#define TH_PREFILL_OPS(STR)                                                                \
  asm volatile(STR                                                                         \
               :                                                                           \
               : "v"(qp), "v"(op), "v"(lim), "v"(klane), "v"(vlane), "v"(krow), "v"(kcol), \
                 "v"(vrow), "v"(vcol), "s"(kbase), "s"(vbase), "s"(kvlast), "s"(nb),       \
                 "s"(jd), "s"(lds_base), "s"(wave2k), "s"(scale_log2), "s"(lratio), "s"(ok), \
                 "s"(jl)                                                                   \
               : TH_PREFILL_ASM_CLOBBERS, "vcc", "scc", "m0", "memory")
  if constexpr (DT == kBF16) TH_PREFILL_OPS(TH_PREFILL_ASM_BF16); else TH_PREFILL_OPS(TH_PREFILL_ASM_F16);
#undef TH_PREFILL_OPS
}

// Grid = ceil(seq_len/256) * batch * num_heads workgroups of 512 threads, heavy
// (late) query blocks first.
template <int DT>
__global__ void __launch_bounds__(NT, 1)
attn_prefill_asm(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
                 const uint16_t* __restrict__ V, uint16_t* __restrict__ O, uint32_t batch,
                 uint32_t seq_len, uint32_t start_pos, uint32_t max_seq, uint32_t nh,
                 uint32_t nkv, float scale_log2) {
  const uint32_t nqb = (seq_len + BQ - 1) / BQ;
  uint32_t bh, qb;
  prefill_work(blockIdx.x, batch, nh, nkv, nqb, bh, qb);
  prefill_tile<DT>(Q, K, V, O, seq_len, start_pos, max_seq, nh, nkv, scale_log2, bh, qb);
}
}  // namespace pfa
}  // namespace th
