// kernels_attn.hip — split-K fused decode attention over the packed KIVI cache.
//
// Semantics: KiviCache::attention / RagSession::attention (reference src/cache.rs:224-279,
// src/prefix.rs:228-289, src/attention.rs:47-105). Token order is global: keys
// [0,kq) packed | [kq,seq) fp32 residual | [seq,seq+L) suffix; values [0,vq) packed |
// [vq,seq) fp32 window | suffix. Each split computes its own softmax max and the splits
// are merged exactly by log-sum-exp, so results equal the reference's two-pass softmax
// within f32 rounding (never bitwise). Logits are kept in base-2 units
// (q pre-multiplied by scale*log2(e)) so every exponential is one v_exp_f32.
//
// The split kernels write one workspace of partials (m, l, acc[D]) per (unit, split, head);
// k_attn_merge combines them:
//  * k_attn_mfma<BITS,NRS,D> — every 64-token chunk whose keys AND values are packed, for
//    head_dim 64/128/192/256, G = 32 or a multiple of 64, bits 2/4/8, any GQA (rows of 4
//    heads, NRS row sets per workgroup, head groups beyond that). Both contractions run on
//    the matrix cores (v_mfma_f32_4x4x4_16b_f16; the non-code operand as f16 hi + lo, about
//    22 significant bits; the codes exact):
//      logits[h][t] = bias_g[h] + sum_d (q[h][d]*scale_g[d]) * code[d][t]
//      out[h][d]   += sum_t (w[h][t]*scale_t[cg]) * code[t][d] + sum_t w[h][t]*zero_t[cg]
//    The GQA heads are the 4 MFMA rows; the 16 4x4 blocks tile 64 tokens (keys) or 64
//    channels (values); CBSZ/ABID broadcast lets one A register feed 8 K-steps. A lane owns
//    a token (keys) or D/64 channels (values), and the native layout packs exactly that
//    lane's codes into its words, so a word unpacks into 4-16 MFMA B operands. At head_dim
//    128 the same launch takes the window / suffix chunks (fp32 rows, a quarter chunk per
//    wave); at other head_dims the tokens after the packed chunks run as generic splits in
//    its grid.
//  * k_attn_shared / k_attn_sessions / k_attn_suffix — batched sessions over one shared
//    prefix (the prefix read once for all sessions).
//  * k_attn_generic — every shape the MFMA kernel does not cover, caches with no packed keys
//    yet and the quality guard's fp32 attention: one wavefront per token in the reference's
//    operation order (recon = fma(code, scale, zero); logit = fma(recon, q, logit), channels
//    ascending, src/attention.rs:143-177, 289-300).
#include "common.hpp"
#include "kivi.h"

#include <algorithm>
#include <mutex>

namespace kivi {

// 1.0 that the compiler cannot fold (external linkage, and constant memory is initialised from
// the host): x * kMixOne - hi stays an fma with an f32 and an f16 source, one mixed-precision
// instruction (lo_pair).
__constant__ float kMixOne = 1.0f;

namespace {

constexpr int kThreads = 256;
constexpr int kHeadsPerPass = 4;
constexpr float kLog2e = 1.4426950408889634f;

typedef float v4f __attribute__((ext_vector_type(4)));

struct AttnArgs {
  CacheView c;
  SeqState st;
  uint64_t seq;
  uint64_t total;          // seq + L
  const float* suffix_k;
  const float* suffix_v;
  uint64_t L;
  uint64_t suffix_stride;  // floats between units of the suffix arrays
  const float* query;      // [batch][QH][D]
  uint32_t qh, heads, gq;
  float scale2;            // scale * log2(e)
  // generic splits: tokens [t_begin, total) in splits of S
  uint64_t t_begin;
  uint32_t S;
  uint32_t nsplit_gen;
  // MFMA splits: packed chunks [chunk_begin, chunk_end) in workgroups of 4 waves x kFastCpw
  // chunks (workspace splits 0 .. nsplit_fast-1), then window / suffix chunks
  // [win_begin, win_end), one per workgroup (splits nsplit_fast .. +nsplit_win-1); generic
  // splits, if any, follow.
  uint32_t chunk_begin;
  uint32_t chunk_end;
  uint32_t nsplit_fast;
  uint32_t win_begin, win_end;
  uint32_t nsplit_win;
  uint32_t nsplit_total;   // splits per unit in the workspace
  // query heads in groups of up to 8 (GQA > 8 on the matrix-core path): one workgroup per
  // (unit, head group, split), each writing its group's partial rows. hgroups_fast: the head
  // groups of the packed splits (groups of 16 on the sixteen-head kernel, hgroups otherwise)
  uint32_t hgroups, hgroups_fast;
  uint32_t gshift;         // log2(G) on the matrix-core path (G = 32, 64 or 128 there)
  // packed splits on the 16x16x32 kernels: 1 eight-head (k_attn_wide), 2 sixteen-head
  // (k_attn_wide16)
  uint32_t wide;
  float* ws;               // [units][nsplit_total][gq][D+2]
  // batched sessions (0 otherwise): session count and the strides between consecutive
  // sessions' queries, partials and outputs
  uint32_t nsess;
  // the shared-prefix GEMM covers prefix chunks [0, gemm_end); k_attn_suffix takes the
  // suffixes in nsplit_win runs per session
  uint32_t gemm_end;
  uint64_t q_sess_stride, ws_sess_stride;
  float* out;              // [batch][QH][D]
  uint32_t units;
  // A decode token appended by this launch (RuntimeKv::decode in one launch; null otherwise):
  // the state above already counts it. Token seq-1's key and value rows are read from pend_k /
  // pend_v ([units][D]) instead of the residual and the window (the merge launch writes them
  // there afterwards); with pend_evict, token vq-1 left the window: its row is still in ring
  // slot pend_vslot, and the workgroup whose chunk holds it quantizes it, writes its codes and
  // (scale, zero), and uses them in place of the packed data not yet in memory.
  const float* pend_k;
  const float* pend_v;
  uint32_t pend_vslot;
  uint32_t pend_evict;
};

// Key / value element (token t, channel d) of one unit, wherever it lives. BITS, DD, GG are
// the compile-time shape (0 = read it from the geometry at run time). Branch free: the packed
// and the fp32 candidate are both loaded from clamped, always-valid addresses and blended, so
// unrolled callers keep many loads in flight. Both candidates are finite (arenas are zero
// filled), so the blend returns exactly the selected one.
template <int BITS, int DD, int GG>
__device__ __forceinline__ float key_at(const AttnArgs& a, uint32_t unit, uint64_t t, uint32_t d) {
  const Geometry& g = a.c.geo;
  const uint32_t bits = BITS ? BITS : g.bits, D = DD ? DD : g.D, G = GG ? GG : g.G;
  const uint32_t ppw = 32 / bits, kw = D / ppw;
  const uint64_t kq = a.st.kq;
  // packed candidate
  const uint64_t tp = kq > 0 ? (t < kq ? t : kq - 1) : 0;
  const uint32_t* wp = kq > 0 ? a.c.kcodes + unit * (g.cap * kw) + tp * kw + d / ppw
                              : reinterpret_cast<const uint32_t*>(a.query);
  const float2* sp = kq > 0 ? reinterpret_cast<const float2*>(a.c.kparams + unit * ((g.cap / G) * D * 2)) + (tp / G) * D + d
                            : reinterpret_cast<const float2*>(a.query);
  // fp32 candidate: key residual, else suffix
  const bool res = t < a.seq;
  const uint32_t tr = t >= kq && res ? static_cast<uint32_t>(t - kq) : 0;
  const uint32_t ts = t >= a.seq ? static_cast<uint32_t>(t - a.seq) : 0;
  const float* dp = res || a.suffix_k == nullptr ? a.c.kres + ((uint64_t)unit * g.R + tr) * D + d
                                                 : a.suffix_k + unit * a.suffix_stride + ts * D + d;
  const uint32_t word = *wp;
  const float2 sz = *sp;
  const float dense = *dp;
  const float code = static_cast<float>((word >> code_shift(bits, d % ppw)) & ((1u << bits) - 1u));
  // arithmetic blend (not a select) so the compiler cannot sink either load into a branch
  const float m = t < kq ? 1.f : 0.f;
  return fmaf(fmaf(code, sz.x, sz.y), m, dense * (1.f - m));  // exact for m in {0, 1}
}

template <int BITS, int DD, int GG>
__device__ __forceinline__ float value_at(const AttnArgs& a, uint32_t unit, uint64_t t, uint32_t d) {
  const Geometry& g = a.c.geo;
  const uint32_t bits = BITS ? BITS : g.bits, D = DD ? DD : g.D, G = GG ? GG : g.G;
  const uint32_t ppw = 32 / bits, vw = kValueBlock / ppw;
  const uint64_t vq = a.st.vq;
  const uint64_t tp = vq > 0 ? (t < vq ? t : vq - 1) : 0;
  const uint64_t tb = tp / kValueBlock;
  const uint32_t tt = tp % kValueBlock;
  const uint32_t* wp = vq > 0 ? a.c.vcodes + unit * ((g.cap / kValueBlock) * D * vw) + (tb * D + d) * vw + tt / ppw
                              : reinterpret_cast<const uint32_t*>(a.query);
  const float2* sp = vq > 0 ? reinterpret_cast<const float2*>(a.c.vparams + unit * (g.cap * (D / G) * 2)) +
                                  (tb * (D / G) + d / G) * kValueBlock + tt
                            : reinterpret_cast<const float2*>(a.query);
  const bool win = t < a.seq;
  uint32_t slot = a.st.vhead + (t >= vq && win ? static_cast<uint32_t>(t - vq) : 0);  // < 2R
  if (slot >= g.R) slot -= g.R;
  const uint32_t ts = t >= a.seq ? static_cast<uint32_t>(t - a.seq) : 0;
  const float* dp = win || a.suffix_v == nullptr ? a.c.vring + ((uint64_t)unit * g.R + slot) * D + d
                                                 : a.suffix_v + unit * a.suffix_stride + ts * D + d;
  const uint32_t word = *wp;
  const float2 sz = *sp;
  const float dense = *dp;
  const float code = static_cast<float>((word >> code_shift(bits, tt % ppw)) & ((1u << bits) - 1u));
  const float m = t < vq ? 1.f : 0.f;
  return fmaf(fmaf(code, sz.x, sz.y), m, dense * (1.f - m));  // exact for m in {0, 1}
}

// DPP exchanges inside rows of 16 lanes (every lane active): quad_perm xor 1 and xor 2, then
// the mirrors that pair each lane with the other half of its 8- and 16-lane group.
template <int CTRL>
__device__ __forceinline__ float dpp_row(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}
// max (MAX) or min over each 16-lane row, in every lane of the row
template <bool MAX>
__device__ __forceinline__ float row_reduce(float v) {
  v = MAX ? fmaxf(v, dpp_row<0xB1>(v)) : fminf(v, dpp_row<0xB1>(v));
  v = MAX ? fmaxf(v, dpp_row<0x4E>(v)) : fminf(v, dpp_row<0x4E>(v));
  v = MAX ? fmaxf(v, dpp_row<0x141>(v)) : fminf(v, dpp_row<0x141>(v));
  v = MAX ? fmaxf(v, dpp_row<0x140>(v)) : fminf(v, dpp_row<0x140>(v));
  return v;
}
__device__ __forceinline__ float lane_value(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
// max over the wave (every lane active): rows by DPP, then the four rows' maxima by readlane,
// in place of six dependent LDS-path shuffles
__device__ __forceinline__ float warp_max(float v) {
  v = row_reduce<true>(v);
  return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}
__device__ __forceinline__ float warp_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// ------------------------------------------------------------------ generic splits
// One workgroup per (unit, split) over tokens [t_begin, total). LDS: q [gq][D], logits/weights
// [gq][S]. Instantiated for every shape (BITS = DD = GG = 0) and, with the shape fixed, for the
// tail of the MFMA path (the fp32 window, the session suffix and a partial last chunk).
template <int BITS, int DD, int GG>
__device__ __forceinline__ void generic_split(const AttnArgs& a, uint32_t unit, uint32_t split,
                                              float* lds) {
  const Geometry& g = a.c.geo;
  const uint32_t D = DD ? DD : g.D, gq = a.gq, S = a.S;
  const uint32_t b = unit / a.heads, kvh = unit % a.heads;
  float* q_lds = lds;               // [gq][D], pre-scaled to base-2 logits
  float* w_lds = lds + gq * D;      // [gq][S]
  const uint64_t t0 = a.t_begin + (uint64_t)split * S;
  const uint32_t ntok = static_cast<uint32_t>(std::min<uint64_t>(S, a.total - t0));

  for (uint32_t i = threadIdx.x; i < gq * D; i += blockDim.x) {
    const uint32_t h = i / D, d = i % D;
    q_lds[i] = a.query[((uint64_t)b * a.qh + kvh * gq + h) * D + d];
  }
  __syncthreads();

  // Logits: one wavefront per token (lanes over channels, so every load is coalesced), four
  // tokens per iteration so their loads are in flight together; heads in passes of 4.
  const uint32_t lane = threadIdx.x % 64, wave = threadIdx.x / 64, nwave = blockDim.x / 64;
  const uint32_t passes = (gq + kHeadsPerPass - 1) / kHeadsPerPass;
  for (uint32_t k0 = wave * 4; k0 < ntok; k0 += nwave * 4) {
    for (uint32_t pass = 0; pass < passes; ++pass) {
      const uint32_t h0 = pass * kHeadsPerPass;
      const uint32_t nh = std::min<uint32_t>(kHeadsPerPass, gq - h0);
      float acc[4][kHeadsPerPass] = {};
      for (uint32_t d0 = 0; d0 < D; d0 += 64) {
        const uint32_t d = std::min<uint32_t>(d0 + lane, D - 1);  // clamped: loads stay unconditional
        const float live_d = d0 + lane < D ? 1.f : 0.f;
        float kv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t k = std::min<uint32_t>(k0 + j, ntok - 1);
          kv[j] = key_at<BITS, DD, GG>(a, unit, t0 + k, d) * live_d;
        }
#pragma unroll
        for (int h = 0; h < kHeadsPerPass; ++h) {
          const float qd = h < (int)nh ? q_lds[(h0 + h) * D + d] : 0.f;
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[j][h] = fmaf(kv[j], qd, acc[j][h]);
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int h = 0; h < kHeadsPerPass; ++h) {
          const float v = warp_sum(acc[j][h]);
          if (lane == 0 && h < (int)nh && k0 + j < ntok) w_lds[(h0 + h) * S + k0 + j] = v * a.scale2;
        }
    }
  }
  __syncthreads();

  // Per-head max and exp2-sum over the split (one wavefront per head).
  float* part = a.ws + ((uint64_t)unit * a.nsplit_total + a.nsplit_fast + a.nsplit_win + split) * gq * (D + 2);
  for (uint32_t h = wave; h < gq; h += blockDim.x / 64) {
    float m = -INFINITY;
    for (uint32_t k = lane; k < ntok; k += 64) m = fmaxf(m, w_lds[h * S + k]);
    m = warp_max(m);
    float l = 0.f;
    for (uint32_t k = lane; k < ntok; k += 64) {
      const float w = exp2f(w_lds[h * S + k] - m);
      w_lds[h * S + k] = w;
      l += w;
    }
    l = warp_sum(l);
    if (lane == 0) {
      part[h * (D + 2) + D] = m;
      part[h * (D + 2) + D + 1] = l;
    }
  }
  __syncthreads();

  // Value mix: one (channel, head pass) per thread, tokens ascending, 8 loads in flight.
  for (uint32_t idx = threadIdx.x; idx < D * passes; idx += blockDim.x) {
    const uint32_t d = idx % D, pass = idx / D;
    const uint32_t h0 = pass * kHeadsPerPass;
    const uint32_t nh = std::min<uint32_t>(kHeadsPerPass, gq - h0);
    float acc[kHeadsPerPass] = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t k0 = 0; k0 < ntok; k0 += 8) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = value_at<BITS, DD, GG>(a, unit, t0 + std::min<uint32_t>(k0 + j, ntok - 1), d);
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int h = 0; h < kHeadsPerPass; ++h) {
          const float wj = k0 + j < ntok ? w_lds[(h0 + h) * S + std::min<uint32_t>(k0 + j, ntok - 1)] : 0.f;
          acc[h] = fmaf(v[j], wj, acc[h]);
        }
    }
#pragma unroll
    for (int h = 0; h < kHeadsPerPass; ++h)
      if (h < (int)nh) part[(h0 + h) * (D + 2) + d] = acc[h];
  }
}

template <int BITS, int DD, int GG>
__global__ void __launch_bounds__(kThreads) k_attn_generic(AttnArgs a) {
  extern __shared__ float lds[];
  const uint32_t unit = blockIdx.x / a.nsplit_gen;
  generic_split<BITS, DD, GG>(a, unit, blockIdx.x % a.nsplit_gen, lds);
}

// ------------------------------------------------------------------ MFMA splits

constexpr int kFastCpw = 8;  // chunks (64 tokens) per wave in the MFMA kernel
constexpr int kCpw6MaxBits = 4;
// Chunks per wave per instantiation: the eight-head 2- and 4-bit ones take 6, so their logit
// rows (49.7 KB of LDS per workgroup instead of 66 KB) let three workgroups share a CU, as
// their registers allow (C3 4-bit: 51.8 us against 55.4 us with 8; 8-bit is slower with 6).
constexpr int fast_cpw(int bits, int nrs) { return nrs == 2 && bits <= kCpw6MaxBits ? 6 : kFastCpw; }
// Packed workgroups a launch aims for at least (one per CU): below it, waves take fewer than
// kFastCpw chunks. More workgroups than that with fewer chunks each measured slower (4-bit,
// 8 units x 131072 tokens: 1024 workgroups of 4 chunks per wave 62 us, 512 of 8 55 us).
constexpr uint32_t kFastGroups = 256;
constexpr int kRowPad = 4;  // floats of padding per logit row (LDS bank spread)
constexpr int kRowStride1 = 64 + kRowPad;  // logits row stride of the one-chunk (MIXED) path

// v_mfma_f32_4x4x1_16B with CBSZ=3: blocks 0-7 take A from block ABID, blocks 8-15 from
// block 8+ABID. ABID must be an immediate; the switch folds away once loops are unrolled.
__device__ __forceinline__ v4f mfma_bcast(float a, float b, v4f c, int abid) {
  switch (abid) {
    case 0: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 3, 0, 0);
    case 1: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 3, 1, 0);
    case 2: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 3, 2, 0);
    case 3: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 3, 3, 0);
    case 4: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 3, 4, 0);
    case 5: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 3, 5, 0);
    case 6: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 3, 6, 0);
    default: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 3, 7, 0);
  }
}

// Sum over lanes 4, 8 and 16 apart (the block index inside a 32-lane half): ds_swizzle in
// bit-mask mode, xor within 32 lanes.
__device__ __forceinline__ float sum_over_blocks(float v) {
  v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1F | (4 << 10)));
  v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1F | (8 << 10)));
  v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1F | (16 << 10)));
  return v;
}

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));

// v_mfma_f32_4x4x4_16b_f16 with CBSZ=3: 16 blocks of D[4x4] += A[4x4] * B[4x4] (K = 4),
// blocks 0-7 taking A from block ABID and blocks 8-15 from block 8+ABID. Lane l holds
// B[k][l%4] of block l/4 for k = 0..3 and gets D[i][l%4] of its block in register i.
__device__ __forceinline__ v4f mfma16(h4 a, h4 b, v4f c, int abid) {
  switch (abid) {
    case 0: return __builtin_amdgcn_mfma_f32_4x4x4f16(a, b, c, 3, 0, 0);
    case 1: return __builtin_amdgcn_mfma_f32_4x4x4f16(a, b, c, 3, 1, 0);
    case 2: return __builtin_amdgcn_mfma_f32_4x4x4f16(a, b, c, 3, 2, 0);
    case 3: return __builtin_amdgcn_mfma_f32_4x4x4f16(a, b, c, 3, 3, 0);
    case 4: return __builtin_amdgcn_mfma_f32_4x4x4f16(a, b, c, 3, 4, 0);
    case 5: return __builtin_amdgcn_mfma_f32_4x4x4f16(a, b, c, 3, 5, 0);
    case 6: return __builtin_amdgcn_mfma_f32_4x4x4f16(a, b, c, 3, 6, 0);
    default: return __builtin_amdgcn_mfma_f32_4x4x4f16(a, b, c, 3, 7, 0);
  }
}

template <int BITS>
struct CodeUnit {
  static constexpr int kExp = BITS == 2 ? -1 : BITS == 4 ? -9 : 0;
};

// Elements 4k .. 4k+3 of a native code word (layout of code_shift) as an exact f16 MFMA
// operand times 2^kExp. 2-bit: masking with 0x33333333 (and after a shift by 2) leaves one
// code per nibble, elements 0-7 (8-15) in nibble order; a nibble p < 4 read as fp4 e2m1 is
// exactly p/2, and v_cvt_scalef32_pk_f16_fp4 converts the two nibbles of one byte. 4-bit:
// masking with 0x0F0F0F0F after a shift by 4k leaves elements 4k..4k+3 one per byte; a byte
// p < 16 read as fp8 e4m3 is exactly p * 2^-9 (subnormals and the first binade are evenly
// spaced). 8-bit: v_perm_b32 places each byte under the f16 exponent of 1024 (0x64), giving
// 1024 + p exactly, and a packed f16 subtraction removes the 1024.
template <int BITS>
__device__ __forceinline__ h4 codes4(uint32_t w, int k) {
  if constexpr (BITS == 2) {
    const uint32_t m = k < 2 ? (w & 0x33333333u) : ((w >> 2) & 0x33333333u);
    h2 a, b;
    if (k % 2 == 0) {
      a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(m, 1.0f, 0);
      b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(m, 1.0f, 1);
    } else {
      a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(m, 1.0f, 2);
      b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(m, 1.0f, 3);
    }
    return h4{a.x, a.y, b.x, b.y};
  } else if constexpr (BITS == 4) {
    const int m = static_cast<int>((w >> (4 * k)) & 0x0F0F0F0Fu);
    const h2 a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(m, 1.0f, false);
    const h2 b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(m, 1.0f, true);
    return h4{a.x, a.y, b.x, b.y};
  } else {
    const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, w, 0x04010400u);  // bytes 0, 1
    const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, w, 0x04030402u);  // bytes 2, 3
    const h2 bias = {(_Float16)1024.0f, (_Float16)1024.0f};
    const h2 x = __builtin_bit_cast(h2, lo) - bias;
    const h2 y = __builtin_bit_cast(h2, hi) - bias;
    return h4{x.x, x.y, y.x, y.y};
  }
}

// The lo halves of two values x, y whose f16 hi halves are the packed pair `hi`:
// (f16(x - hi.x), f16(y - hi.y)), each rounded to nearest from the exact difference: two
// mixed-precision fmas and one packed conversion, in place of two conversions back to f32, two
// subtractions and the packed conversion.
__device__ __forceinline__ uint32_t lo_pair(float x, float y, uint32_t hi) {
  const h2 h = __builtin_bit_cast(h2, hi);
  const float one = kMixOne;
  h2 l;
  l.x = static_cast<_Float16>(__builtin_fmaf(x, one, -static_cast<float>(h.x)));
  l.y = static_cast<_Float16>(__builtin_fmaf(y, one, -static_cast<float>(h.y)));
  return __builtin_bit_cast(uint32_t, l);
}

// x = hi + lo with hi = f16(x) rounded toward zero and lo = f16(x - hi) rounded to nearest:
// 22 significant bits in two f16 operands, two values per packed conversion (x must be below
// 2^15 in magnitude; the callers scale their operands by a power of two).
__device__ __forceinline__ void split4(const float* x, h4& hi, h4& lo) {
  const uint32_t w01 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(x[0], x[1]));
  const uint32_t w23 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(x[2], x[3]));
  const h2 h01 = __builtin_bit_cast(h2, w01), h23 = __builtin_bit_cast(h2, w23);
  const h2 l01 = __builtin_bit_cast(h2, lo_pair(x[0], x[1], w01));
  const h2 l23 = __builtin_bit_cast(h2, lo_pair(x[2], x[3], w23));
  hi = h4{h01.x, h01.y, h23.x, h23.y};
  lo = h4{l01.x, l01.y, l23.x, l23.y};
}

template <int N>
__device__ __forceinline__ void load_words(const uint32_t* p, uint32_t* w) {
  const uint4* v = reinterpret_cast<const uint4*>(p);
#pragma unroll
  for (int j = 0; j < N / 4; ++j) {
    const uint4 x = v[j];
    w[4 * j] = x.x;
    w[4 * j + 1] = x.y;
    w[4 * j + 2] = x.z;
    w[4 * j + 3] = x.w;
  }
}

// Channel geometry of the matrix-core path for head_dim D (64, 128, 192 or 256): keys in sets
// of up to 128 channels (KS of them), set s's channel blocks of 16 (kb(s): 8, or 4 for a
// 64-channel set) held by blocks 0..kb(s)-1 of each half-wave for the broadcast; values D/64
// channels per lane (channels lane + 64*hv).
template <int D>
struct Chan {
  static constexpr int KS = (D + 127) / 128;
  static constexpr int kb(int s) { return D - 128 * s >= 128 ? 8 : (D - 128 * s) / 16; }
  static constexpr int HV = D / 64;
};

// One chunk's key data for the lane's token: its code words, and the (scale, zero) pairs of
// its half's key group (tokens 32*lc .. +31 of the chunk; the same group for both halves when
// G >= 64) for channels 128*s + 16*la + 4*li .. +3 of each set s (the quad's four lanes hold
// the block's 16 channels between them; quad_bcast shares them; in a 64-channel set the
// blocks la >= 4 repeat blocks la - 4, whose operands are never broadcast).
template <int BITS, int D>
struct KeyWords {
  uint32_t w[D * BITS / 32];
};
template <int D>
struct KeyParams {
  float4 sz[Chan<D>::KS][2];
};
// One chunk's value data: the code words of channels lane + 64*hv, and (scale, zero) of
// tokens 8*la + 2*li, +1 for the channel group of channels 32*lc + 64*hv (value_group; the
// quad holds tokens 8*la .. +7).
template <int BITS, int D>
struct ValueWords {
  uint32_t w[Chan<D>::HV][64 * BITS / 32];
};
template <int D>
struct ValueParams {
  float4 sz[Chan<D>::HV];
};

// Sum of v over each quad, in every lane of it: (v0 + v1) + (v2 + v3) (DPP quad_perm; every
// lane is active here).
__device__ __forceinline__ float quad_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, true));  // [1,0,3,2]
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, true));  // [2,3,0,1]
  return v;
}

// v as held by lane q of each quad (DPP quad_perm broadcast; every lane is active here).
__device__ __forceinline__ float quad_bcast(float v, int q) {
  const int x = __float_as_int(v);
  switch (q) {
    case 0: return __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x00, 0xF, 0xF, true));
    case 1: return __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x55, 0xF, 0xF, true));
    case 2: return __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0xAA, 0xF, 0xF, true));
    default: return __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0xFF, 0xF, 0xF, true));
  }
}

template <int BITS, int D>
__device__ __forceinline__ void load_key_words(const AttnArgs& a, uint32_t unit, uint32_t ch,
                                               uint32_t lane, KeyWords<BITS, D>& kw) {
  constexpr int KW = D * BITS / 32;
  load_words<KW>(a.c.kcodes + unit * a.c.geo.kcodes_unit() + ((uint64_t)ch * 64 + lane) * KW, kw.w);
}
template <int D>
__device__ __forceinline__ void load_key_params(const AttnArgs& a, uint32_t unit, uint32_t ch,
                                                uint32_t la, uint32_t lc, uint32_t li, KeyParams<D>& kp) {
  // the key group of the half's tokens 64*ch + 32*lc .. +31 (G a multiple of 32)
  const uint32_t grp = (64 * ch + 32 * lc) >> a.gshift;
#pragma unroll
  for (int ks = 0; ks < Chan<D>::KS; ++ks) {
    const uint32_t blk = la % Chan<D>::kb(ks);
    const float4* pp = reinterpret_cast<const float4*>(
        a.c.kparams + unit * a.c.geo.kparams_unit() + ((uint64_t)grp * D + 128 * ks + 16 * blk + 4 * li) * 2);
    kp.sz[ks][0] = pp[0];
    kp.sz[ks][1] = pp[1];
  }
}
template <int BITS, int D>
__device__ __forceinline__ void load_value_words(const AttnArgs& a, uint32_t unit, uint32_t tb,
                                                 uint32_t lane, ValueWords<BITS, D>& vw) {
  constexpr int VW = 64 * BITS / 32;
#pragma unroll
  for (int hv = 0; hv < Chan<D>::HV; ++hv)
    load_words<VW>(a.c.vcodes + unit * a.c.geo.vcodes_unit() + ((uint64_t)tb * D + lane + 64 * hv) * VW,
                   vw.w[hv]);
}
// channel group of channels 32*lc + 64*hv .. +31 (the lane's channels lane + 64*hv)
__device__ __forceinline__ uint32_t value_group(const AttnArgs& a, uint32_t lc, uint32_t hv) {
  return (32 * lc + 64 * hv) >> a.gshift;
}
template <int D>
__device__ __forceinline__ void load_value_params(const AttnArgs& a, uint32_t unit, uint32_t tb,
                                                  uint32_t la, uint32_t lc, uint32_t li, ValueParams<D>& vp) {
  const uint32_t ncg = D >> a.gshift;
#pragma unroll
  for (int hv = 0; hv < Chan<D>::HV; ++hv)
    vp.sz[hv] = *reinterpret_cast<const float4*>(
        a.c.vparams + unit * a.c.geo.vparams_unit() +
        (((uint64_t)tb * ncg + value_group(a, lc, hv)) * 64 + 8 * la + 2 * li) * 2);
}

// Key-side A operands of one chunk: q * scale (already times 2^e) per (head, channel) of the
// lane's group, split hi/lo, for K-groups of channels 128*s + 16*la + 4k .. +3; bias[h] =
// sum_d q*zero summed over the blocks of the half (the repeated blocks of a 64-channel set add
// 0), times 2^kExp (it enters through an f32 MFMA).
template <int NRS, int D>
struct KeyA {
  h4 hi[NRS][Chan<D>::KS][4], lo[NRS][Chan<D>::KS][4];
  float bias[NRS];
};

template <int BITS, int NRS, int D>
__device__ __forceinline__ void key_operands(const KeyParams<D>& kp, const float (&qv)[NRS][Chan<D>::KS][16],
                                             uint32_t la, KeyA<NRS, D>& A) {
  constexpr float kUnit = CodeUnit<BITS>::kExp == 0 ? 1.0f : CodeUnit<BITS>::kExp == -1 ? 0.5f : 0.001953125f;
#pragma unroll
  for (int rs = 0; rs < NRS; ++rs) {
    float bias = 0.f;
#pragma unroll
    for (int ks = 0; ks < Chan<D>::KS; ++ks) {
      float p[16];
#pragma unroll
      for (int c = 0; c < 16; ++c) {
        const float4 sz = kp.sz[ks][(c % 4) / 2];  // channel c lives in quad lane c / 4
        const float sc = quad_bcast(c % 2 ? sz.z : sz.x, c / 4);
        const float zc = quad_bcast(c % 2 ? sz.w : sz.y, c / 4);
        p[c] = qv[rs][ks][c] * sc;
        if (la < (uint32_t)Chan<D>::kb(ks)) bias = fmaf(qv[rs][ks][c], zc, bias);
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) split4(p + 4 * k, A.hi[rs][ks][k], A.lo[rs][ks][k]);
    }
    A.bias[rs] = sum_over_blocks(bias) * kUnit;
  }
}

// Logits of one chunk for the lane's token (lane = token within the chunk), scaled by
// 2^(e + kExp). Block a2's lanes hold A for channels 128*s + 16*a2 .. +15, so ABID = a2
// broadcasts it to the 8 token blocks of each half; B = the lane token's codes (exact).
template <int BITS, int NRS, int D>
__device__ __forceinline__ void key_mfma(const KeyWords<BITS, D>& kw, const KeyA<NRS, D>& A,
                                         float (&lg)[NRS][4]) {
  constexpr int PPW = 32 / BITS;
  v4f acc[NRS][2];
#pragma unroll
  for (int rs = 0; rs < NRS; ++rs) {
    acc[rs][0] = v4f{0.f, 0.f, 0.f, 0.f};
    acc[rs][1] = v4f{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int ks = 0; ks < Chan<D>::KS; ++ks) {
#pragma unroll
    for (int a2 = 0; a2 < Chan<D>::kb(ks); ++a2) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int c0 = 128 * ks + 16 * a2 + 4 * k;  // first channel of the K-group
        const h4 b = codes4<BITS>(kw.w[c0 / PPW], (c0 % PPW) / 4);
#pragma unroll
        for (int rs = 0; rs < NRS; ++rs) {
          acc[rs][0] = mfma16(A.hi[rs][ks][k], b, acc[rs][0], a2);
          acc[rs][1] = mfma16(A.lo[rs][ks][k], b, acc[rs][1], a2);
        }
      }
    }
  }
#pragma unroll
  for (int rs = 0; rs < NRS; ++rs) {
    acc[rs][0] = mfma_bcast(A.bias[rs], 1.0f, acc[rs][0], 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) lg[rs][i] = acc[rs][0][i] + acc[rs][1][i];
  }
}

// Value-side A operands of one chunk: w * scale * 2^e per (head, token) of the lane's tokens
// 8*la .. +7 and the channel group of channels 32*lc + 64*hv, split hi/lo into K-groups of 4
// tokens. The zero term sum_t w*zero accumulates into zacc (f32 VALU, unscaled).
template <int NRS, int D>
struct ValueA {
  h4 hi[NRS][Chan<D>::HV][2], lo[NRS][Chan<D>::HV][2];  // [rs][hv][tokens 8*la + 4j ..]
};

// The weights w arrive times 2^e already (the exponent offset of the softmax), so zacc and
// the caller's weight sum are in those units too.
template <int NRS, int D>
__device__ __forceinline__ void value_operands(const ValueParams<D>& vp, const float (&w)[NRS][8],
                                               ValueA<NRS, D>& A, float (&zacc)[NRS][Chan<D>::HV]) {
#pragma unroll
  for (int rs = 0; rs < NRS; ++rs) {
#pragma unroll
    for (int hv = 0; hv < Chan<D>::HV; ++hv) {
      float p[8];
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const float4 sz = vp.sz[hv];  // token 8*la + r lives in quad lane r / 2
        const float sc = quad_bcast(r % 2 ? sz.z : sz.x, r / 2);
        const float zc = quad_bcast(r % 2 ? sz.w : sz.y, r / 2);
        p[r] = w[rs][r] * sc;
        zacc[rs][hv] = fmaf(w[rs][r], zc, zacc[rs][hv]);
      }
      split4(p, A.hi[rs][hv][0], A.lo[rs][hv][0]);
      split4(p + 4, A.hi[rs][hv][1], A.lo[rs][hv][1]);
    }
  }
}

// Value mix of one chunk into vacc (lane = channels lane + 64*hv, scaled by 2^(e+kExp)).
// K-group (word q, k) covers tokens q*PPW + 4k .. +3, whose A lives in block t0/8.
template <int BITS, int NRS, int D>
__device__ __forceinline__ void value_mfma(const ValueWords<BITS, D>& vw, const ValueA<NRS, D>& A,
                                           v4f (&vacc)[NRS][Chan<D>::HV]) {
  constexpr int VW = 64 * BITS / 32, PPW = 32 / BITS;
#pragma unroll
  for (int q = 0; q < VW; ++q) {
#pragma unroll
    for (int k = 0; k < PPW / 4; ++k) {
      const int t0 = q * PPW + 4 * k;
      const int a2 = t0 / 8, j = (t0 / 4) % 2;
      h4 b[Chan<D>::HV];
#pragma unroll
      for (int hv = 0; hv < Chan<D>::HV; ++hv) b[hv] = codes4<BITS>(vw.w[hv][q], k);
      // the hi products of every channel set, then the lo ones: consecutive MFMAs use
      // different accumulators where D allows
#pragma unroll
      for (int rs = 0; rs < NRS; ++rs) {
#pragma unroll
        for (int hv = 0; hv < Chan<D>::HV; ++hv) vacc[rs][hv] = mfma16(A.hi[rs][hv][j], b[hv], vacc[rs][hv], a2);
#pragma unroll
        for (int hv = 0; hv < Chan<D>::HV; ++hv) vacc[rs][hv] = mfma16(A.lo[rs][hv][j], b[hv], vacc[rs][hv], a2);
      }
    }
  }
}

// fp32 rows of the chunk path: token t's key row (key residual for kq <= t < seq, session
// suffix for seq <= t < total) and value row (value window ring for vq <= t < seq, suffix
// after). Every other t maps to a valid row whose contribution the caller masks to zero.
__device__ __forceinline__ const float* key_row(const AttnArgs& a, uint32_t unit, uint64_t t) {
  const uint32_t D = a.c.geo.D;
  if (t >= a.seq && t < a.total && a.suffix_k != nullptr)
    return a.suffix_k + unit * a.suffix_stride + (t - a.seq) * D;
  if (a.pend_k != nullptr && t + 1 == a.seq) return a.pend_k + (uint64_t)unit * D;
  const uint64_t r = t >= a.st.kq && t < a.seq ? t - a.st.kq : 0;
  return a.c.kres + ((uint64_t)unit * a.c.geo.R + r) * D;
}
__device__ __forceinline__ const float* value_row(const AttnArgs& a, uint32_t unit, uint64_t t) {
  const uint32_t D = a.c.geo.D, R = a.c.geo.R;
  if (t >= a.seq && t < a.total && a.suffix_v != nullptr)
    return a.suffix_v + unit * a.suffix_stride + (t - a.seq) * D;
  if (a.pend_v != nullptr && t + 1 == a.seq) return a.pend_v + (uint64_t)unit * D;
  uint32_t slot = a.st.vhead + (t >= a.st.vq && t < a.seq ? static_cast<uint32_t>(t - a.st.vq) : 0u);
  if (slot >= R) slot -= R;
  return a.c.vring + ((uint64_t)unit * R + slot) * D;
}

// fp32 key rows of a MIXED wave's quarter: lane l holds token 16*quarter + l%16, channels
// 32*(l/16) .. +31 (every token of the quarter is read once, four lanes per row).
struct KeyRows {
  float4 x[8];
};
__device__ __forceinline__ void load_key_rows(const AttnArgs& a, uint32_t unit, uint64_t t0,
                                              uint32_t quarter, uint32_t lane, KeyRows& kr) {
  const float4* row = reinterpret_cast<const float4*>(key_row(a, unit, t0 + 16 * quarter + lane % 16)) +
                      8 * (lane / 16);
#pragma unroll
  for (int j = 0; j < 8; ++j) kr.x[j] = row[j];
}

// Logit contribution of the quarter's fp32 keys (tokens kq <= t < total), added to lg in the
// packed pass's units, for the lanes of the quarter (l/16 == quarter: token l of the chunk).
// f32 MFMAs without broadcast (v_mfma_f32_4x4x1_16B): block b = l/4 multiplies q of heads
// 0..3 (A, lane 4b+i holds head i) by tokens 16*quarter + 4*(b%4) + c (B, lane 4b+c) at
// channel 32*(b/4) + r; the q values come from the lanes holding them in qv (ds_bpermute),
// and the four channel groups' sums meet across lanes 16 and 32 apart.
template <int NRS>
__device__ __forceinline__ void key_fp32(const AttnArgs& a, uint64_t t0, uint32_t quarter, uint32_t lane,
                                         const float (&qv)[NRS][1][16], const KeyRows& kr,
                                         float unit_scale, float (&lg)[NRS][4]) {
  const uint64_t t = t0 + 16 * quarter + lane % 16;
  const float m = t >= a.st.kq && t < a.total ? unit_scale : 0.f;  // mask times 2^kExp
  // qv of head l%4 at channels 16*la' + c sits in lane 4*la' + l%4 (la' = 2*(l/16) + c/16)
  const int src0 = static_cast<int>(8 * (lane / 16) + lane % 4);
  const int src1 = src0 + 4;
#pragma unroll
  for (int rs = 0; rs < NRS; ++rs) {
    v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < 32; ++r) {
      const float x = (r % 4 == 0 ? kr.x[r / 4].x : r % 4 == 1 ? kr.x[r / 4].y : r % 4 == 2 ? kr.x[r / 4].z : kr.x[r / 4].w) * m;
      const float q = __shfl(qv[rs][0][r % 16], r < 16 ? src0 : src1);
      acc = __builtin_amdgcn_mfma_f32_4x4x1f32(q, x, acc, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = acc[i];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      lg[rs][i] += v;
    }
  }
}

// The quarter's fp32 value rows for channels lane and 64+lane (tokens 16*quarter .. +15, all
// 32 values requested at once). Lane r of each 16 computes row r's address once (vector
// work), and each row's address reaches the wave by readlane, in place of 16 scalar address
// computations with their branches.
struct ValueRows {
  float b[16][2];
};
__device__ __forceinline__ void load_value_rows(const AttnArgs& a, uint32_t unit, uint64_t t0,
                                                uint32_t quarter, uint32_t lane, ValueRows& vr) {
  const uint64_t mine = reinterpret_cast<uint64_t>(value_row(a, unit, t0 + 16 * quarter + lane % 16));
  const uint32_t lo = static_cast<uint32_t>(mine), hi = static_cast<uint32_t>(mine >> 32);
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    // readlane returns int: each word is taken as uint32_t before widening, or a low word with
    // its top bit set would sign-extend over the high word
    const uint64_t p = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(hi, r) << 32) |
                       (uint64_t)(uint32_t)__builtin_amdgcn_readlane(lo, r);
    const float* row = reinterpret_cast<const float*>(p);
    vr.b[r][0] = row[lane];
    vr.b[r][1] = row[lane + 64];
  }
}

// Value contribution of the chunk's fp32 values (tokens vq <= t < total) among tokens
// 16*quarter .. +15, for channels lane and 64+lane, in the packed pass's units: A = w * wscale
// for the lane's tokens 8*la + r (0 for other tokens), broadcast from block t/8; B = the
// token's value row.
template <int NRS>
__device__ __forceinline__ void value_fp32(const AttnArgs& a, uint64_t t0, uint32_t quarter,
                                           uint32_t la, const float* wrow, const float (&moff)[NRS],
                                           float kout, float wscale, const ValueRows& vr,
                                           v4f (&vacc)[NRS][2]) {
  // A: lanes of block la hold the weights of tokens 16*quarter + 8*(la%2) + r, so the
  // quarter's 16 tokens sit in blocks 0 and 1 (ABID 0, 1) whatever the quarter
  const uint32_t tq = 16 * quarter + 8 * (la % 2);
  float am[NRS][8];
#pragma unroll
  for (int rs = 0; rs < NRS; ++rs) {
    const float4* lp = reinterpret_cast<const float4*>(wrow + rs * 4 * kRowStride1 + tq);
    const float4 x0 = lp[0], x1 = lp[1];
    const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const uint64_t t = t0 + tq + r;
      const float m = t >= a.st.vq && t < a.total ? wscale : 0.f;
      am[rs][r] = __builtin_amdgcn_exp2f(fmaf(xs[r], kout, -moff[rs])) * m;
    }
  }
#pragma unroll
  for (int r = 0; r < 16; ++r)
#pragma unroll
    for (int rs = 0; rs < NRS; ++rs) {
      vacc[rs][0] = mfma_bcast(am[rs][r % 8], vr.b[r][0], vacc[rs][0], r / 8);
      vacc[rs][1] = mfma_bcast(am[rs][r % 8], vr.b[r][1], vacc[rs][1], r / 8);
    }
}

// The value row evicted by a decode token appended in the same launch (pend_evict): lane
// holds channels lane and 64+lane, and (min, scale) of their 32-channel groups lc and lc+2,
// computed as the value quantizer does (src/quant.rs:349-375, 453-472).
struct EvictRow {
  float x[2], mn[2], sc[2];
};
__device__ __forceinline__ uint32_t evict_code(float x, float zero, float scale, float levels) {
  if (scale == 0.0f) return 0u;
  float r = rintf((x - zero) / scale);
  if (r < 0.0f) {
    r = 0.0f;
  } else if (r > levels) {
    r = levels;
  }
  return static_cast<uint32_t>(r);
}
// Group min / max over the 32 lanes of each half-wave; returns the row's largest scale and
// largest |x| (whole wave).
__device__ __forceinline__ void evict_groups(EvictRow& e, float levels, float& smax, float& amax) {
  smax = 0.f;
  amax = 0.f;
  const bool low = __lane_id() < 32;
#pragma unroll
  for (int hv = 0; hv < 2; ++hv) {
    // min and max over each half-wave: rows by DPP, then the half's two rows by readlane
    float mn = row_reduce<false>(e.x[hv]), mx = row_reduce<true>(e.x[hv]);
    mn = low ? fminf(lane_value(mn, 0), lane_value(mn, 16)) : fminf(lane_value(mn, 32), lane_value(mn, 48));
    mx = low ? fmaxf(lane_value(mx, 0), lane_value(mx, 16)) : fmaxf(lane_value(mx, 32), lane_value(mx, 48));
    const float fz = lane_group_first_zero(e.x[hv], 32);  // a zero minimum: the first zero's sign
    if (mn == 0.f) mn = fz;
    const float span = mx - mn;
    e.mn[hv] = mn;
    e.sc[hv] = span == 0.0f ? 0.0f : span / levels;
    smax = fmaxf(smax, e.sc[hv]);
    amax = fmaxf(amax, fmaxf(fabsf(mn), fabsf(mx)));
  }
  smax = fmaxf(lane_value(smax, 0), lane_value(smax, 32));
  amax = fmaxf(lane_value(amax, 0), lane_value(amax, 32));
}

// One workgroup = 4 waves; wave w of split s owns packed chunks [s*4*CPW + w*CPW, +CPW) of its
// unit (chunks whose 64 keys and 64 values are all packed). D = 128, G = 32. Per chunk the
// operands are prepared from the (scale, zero) registers first, then the next chunk's data
// is requested into the same registers while this chunk's MFMAs run (code words are
// double-buffered). EARLY (one chunk per wave, launches of a few hundred workgroups such as a
// decode step, where every memory round trip is on the critical path): the chunk's value
// data and fp32 rows are requested with its key data at the start, so the wave waits for
// memory once.
template <int BITS, int NRS, int CPW, bool MIXED, int D, bool EARLY = false>
__device__ __forceinline__ void mfma_split(const AttnArgs& a, uint32_t unit, uint32_t split,
                                           uint32_t hg, float* lds) {
  static_assert(!MIXED || D == 128, "window / suffix chunks are taken at head_dim 128 only");
  static_assert(!EARLY || CPW == 1, "early requests cover one chunk per wave");
  constexpr int KS = Chan<D>::KS, HV = Chan<D>::HV;
  constexpr int ROW = CPW * 64 + kRowPad;  // logits row stride (floats)
  constexpr int NH = 4 * NRS;              // padded heads per unit
  const uint32_t b = unit / a.heads, kvh = unit % a.heads;
  // the wave index as a wave-uniform value: the chunk, quarter and row addresses derived from
  // it are then scalar (a MIXED wave's fp32 row addresses otherwise take divergent branches)
  const uint32_t lane = threadIdx.x % 64, wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  const uint32_t la = (lane % 32) / 4;  // block within a half-wave
  const uint32_t li = lane % 4;         // MFMA row = head within the row set
  const uint32_t lc = lane / 32;        // half-wave: key group / value channel group parity
  const uint32_t gq = a.gq;
  float* wl = lds + wave * NH * ROW;    // this wave's logits [NH][ROW]

  // Packed launch: chunks are dealt round-robin over the unit's waves (wave slot =
  // split*4 + wave, stride = all slots). MIXED launch (CPW = 1): workgroup `split` takes one
  // chunk and wave w its tokens 16w .. 16w+15 (the other tokens' logits are masked), so the
  // latency-bound fp32 rows are spread over four waves.
  const uint32_t c_lo = MIXED ? a.win_begin : a.chunk_begin;
  const uint32_t c_hi = MIXED ? a.win_end : a.chunk_end;
  const uint32_t nsplit = MIXED ? a.nsplit_win : a.nsplit_fast;
  const uint32_t split_base = MIXED ? a.nsplit_fast : 0u;
  const int32_t slots = MIXED ? static_cast<int32_t>(nsplit) : static_cast<int32_t>(nsplit * 4);
  const int32_t slot = MIXED ? static_cast<int32_t>(split) : static_cast<int32_t>(split * 4 + wave);
  const int32_t span = static_cast<int32_t>(c_hi - c_lo);
  const int32_t nch = std::min<int32_t>(CPW, std::max<int32_t>(0, (span - slot + slots - 1) / slots));
  auto chunk_of = [&](int32_t k) { return static_cast<int32_t>(c_lo) + slot + k * slots; };
  const uint32_t quarter = MIXED ? wave : 0;
  const uint64_t kq = a.st.kq, vq = a.st.vq, total = a.total;
  const int32_t lastk = static_cast<int32_t>((kq - 1) / 64);  // kq > 0 on this path
  const int32_t lastv = vq > 0 ? static_cast<int32_t>((vq - 1) / 64) : 0;

  // The first chunk's key data are requested before anything else, so their latency
  // overlaps the query loads and the range set-up.
  KeyParams<D> kp;
  KeyWords<BITS, D> kw0, kw1;
  if (nch > 0) {
    const int32_t k0 = std::min(chunk_of(0), lastk);
    load_key_params<D>(a, unit, k0, la, lc, li, kp);
    load_key_words<BITS, D>(a, unit, k0, lane, kw0);
  }
  // MIXED (one chunk, tw): its fp32 key rows are requested with the packed data, and its fp32
  // value rows as soon as the logits are done, so the workgroup's memory round trips overlap
  // (these workgroups are on the critical path of short launches such as a decode step)
  const uint64_t tw = (uint64_t)chunk_of(0) * 64;
  const bool key_rows = MIXED && nch > 0 && tw + 64 > kq && tw < total;
  const bool value_rows = MIXED && nch > 0 && tw + 16 * quarter + 16 > vq && tw + 16 * quarter < total;
  KeyRows krw;
  ValueRows vrw;
  ValueParams<D> vp;
  ValueWords<BITS, D> vw0, vw1;
  if constexpr (EARLY) {
    if (nch > 0) {
      const int32_t v0 = std::min(chunk_of(0), lastv);
      load_value_params<D>(a, unit, v0, la, lc, li, vp);
      load_value_words<BITS, D>(a, unit, v0, lane, vw0);
    }
    if constexpr (MIXED) {
      if (key_rows) load_key_rows(a, unit, tw, quarter, lane, krw);
      if (value_rows) load_value_rows(a, unit, tw, quarter, lane, vrw);
    }
  }

  // a decode token appended by this launch evicts token vq-1 from the window: its row
  EvictRow er{};
  if (D == 128 && a.pend_evict) {
    const float* row = a.c.vring + ((uint64_t)unit * a.c.geo.R + a.pend_vslot) * D;
    er.x[0] = row[lane];
    er.x[1] = row[lane + 64];
  }

  // q in base-2 logit units for the lane's head, channels 128*s + 16*la .. +15 of each set s
  // (0 for padded heads; D = 64 repeats blocks la - 4 in blocks la >= 4).
  float qv[NRS][KS][16];
  float qmax = 0.f;
#pragma unroll
  for (int rs = 0; rs < NRS; ++rs) {
    const uint32_t h = hg * NH + rs * 4 + li;  // query head within the unit (head group hg)
    const float s = h < gq ? a.scale2 : 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const float* qp =
          a.query + ((uint64_t)b * a.qh + kvh * gq + min(h, gq - 1)) * D + 128 * ks + 16 * (la % Chan<D>::kb(ks));
#pragma unroll
      for (int r = 0; r < 16; r += 4) {
        const float4 v = *reinterpret_cast<const float4*>(qp + r);
        qv[rs][ks][r] = v.x * s;
        qv[rs][ks][r + 1] = v.y * s;
        qv[rs][ks][r + 2] = v.z * s;
        qv[rs][ks][r + 3] = v.w * s;
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) qmax = fmaxf(qmax, fabsf(qv[rs][ks][r]));
    }
  }
  // Power-of-two operand ranges: every key A operand |q * scale| * 2^ek and every value A
  // operand |w * scale| * 2^ev (w <= 1) stays below 2^15, from the unit's largest scales.
  qmax = warp_max(qmax);
  float kmax, vmax_all;  // the unit's largest key and value scales
  unit_scale_max(a.c, unit, kmax, vmax_all);
  constexpr float kLevels = static_cast<float>((1 << BITS) - 1);
  const int ek = std::min(60, std::max(-100, 15 - __builtin_amdgcn_frexp_expf(qmax * kmax)));
  constexpr int kExp = CodeUnit<BITS>::kExp;
  const float kfac = ldexpf(1.f, ek);
  const float kout = ldexpf(1.f, -ek - kExp);
#pragma unroll
  for (int rs = 0; rs < NRS; ++rs)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int r = 0; r < 16; ++r) qv[rs][ks][r] *= kfac;

  // ---------------- phase 1: logits of every owned chunk into LDS (scaled by 2^(ek+kExp))
  // A chunk's keys are packed for t < kq and fp32 after; packed arrays hold zero codes and
  // zero (scale, zero) beyond kq (and vq), so each pass contributes nothing outside its range
  // and the fp32 passes mask theirs. Tokens past `total` get logit -inf.
  constexpr float kUnit = kExp == 0 ? 1.0f : kExp == -1 ? 0.5f : 0.001953125f;
  float mx[NRS][4];
#pragma unroll
  for (int rs = 0; rs < NRS; ++rs)
#pragma unroll
    for (int i = 0; i < 4; ++i) mx[rs][i] = -INFINITY;
  {
    KeyA<NRS, D> A;
    auto step = [&](int k, const KeyWords<BITS, D>& cur, KeyWords<BITS, D>& next) {
      const uint64_t t0 = (uint64_t)chunk_of(k) * 64;
      const bool packed = !MIXED || t0 < kq;
      if (packed) key_operands<BITS, NRS, D>(kp, qv, la, A);
      // unconditional (clamped to packed chunks; the last step re-reads an L2-resident chunk)
      if constexpr (CPW > 1) {
        const int32_t kn = std::min(chunk_of(std::min(k + 1, nch - 1)), lastk);
        load_key_params<D>(a, unit, kn, la, lc, li, kp);
        load_key_words<BITS, D>(a, unit, kn, lane, next);
      }
      float lg[NRS][4];
#pragma unroll
      for (int rs = 0; rs < NRS; ++rs)
#pragma unroll
        for (int i = 0; i < 4; ++i) lg[rs][i] = 0.f;
      if (packed) key_mfma<BITS, NRS, D>(cur, A, lg);
      if constexpr (MIXED) {
        if (key_rows) {  // t0 == tw
          if constexpr (!EARLY) load_key_rows(a, unit, tw, quarter, lane, krw);
          key_fp32<NRS>(a, t0, quarter, lane, qv, krw, kUnit, lg);
        }
      }
      const bool live = !MIXED || (t0 + lane < total && lane / 16 == quarter);
#pragma unroll
      for (int rs = 0; rs < NRS; ++rs)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float v = live ? lg[rs][i] : -INFINITY;
          wl[(rs * 4 + i) * ROW + k * 64 + lane] = v;
          mx[rs][i] = fmaxf(mx[rs][i], v);
        }
    };
    for (int k = 0; k < nch; k += 2) {
      step(k, kw0, kw1);
      if (k + 1 < nch) step(k + 1, kw1, kw0);
    }
  }
  // wave max per head; each lane keeps the max of its own MFMA row (true base-2 units)
  if constexpr (MIXED && !EARLY) {
    if (value_rows) load_value_rows(a, unit, tw, quarter, lane, vrw);
  }
  float mrow[NRS];
#pragma unroll
  for (int rs = 0; rs < NRS; ++rs) {
    float mall[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) mall[i] = warp_max(mx[rs][i]) * kout;
    mrow[rs] = li == 0 ? mall[0] : li == 1 ? mall[1] : li == 2 ? mall[2] : mall[3];
  }
  // the value operands' range: the unit's largest value scale, raised by the evicted row's
  // quantization when a decode token is appended by this launch (as the append would have);
  // taken after the logits, so the evicted row's load is not waited for before them
  float vmax = vmax_all;
  float ev_scale = 0.f, ev_amax = 0.f;  // the evicted row's largest scale and |x|
  if (D == 128 && a.pend_evict) {
    evict_groups(er, kLevels, ev_scale, ev_amax);
    vmax = fmaxf(vmax, ev_scale);
  }
  const int ev = std::min(60, std::max(-100, 15 - __builtin_amdgcn_frexp_expf(vmax)));
  const float vfac = ldexpf(1.f, ev);
  const float vout = ldexpf(1.f, -ev - kExp);
  // exponent offset: the row max, or 0 when every logit of the row is -inf (a MIXED wave whose
  // quarter lies past `total`), so the weights are 0 rather than NaN
  float moff[NRS];
#pragma unroll
  for (int rs = 0; rs < NRS; ++rs) moff[rs] = mrow[rs] == -INFINITY ? 0.f : mrow[rs];
  // the packed value pass takes its weights times 2^ev straight from the exponential
  float evoff[NRS];
#pragma unroll
  for (int rs = 0; rs < NRS; ++rs) evoff[rs] = static_cast<float>(ev) - moff[rs];
  const float vinv = ldexpf(1.f, -ev);

  // ---------------- phase 2: value mix
  v4f vacc[NRS][HV];
  float zacc[NRS][HV];
  float lsum[NRS];
#pragma unroll
  for (int rs = 0; rs < NRS; ++rs) {
#pragma unroll
    for (int hv = 0; hv < HV; ++hv) {
      vacc[rs][hv] = v4f{0.f, 0.f, 0.f, 0.f};
      zacc[rs][hv] = 0.f;
    }
    lsum[rs] = 0.f;
  }
  {
    ValueA<NRS, D> A;
    auto step = [&](int k, ValueWords<BITS, D>& cur, ValueWords<BITS, D>& next) {
      const uint64_t t0 = (uint64_t)chunk_of(k) * 64;
      const bool packed = !MIXED || t0 < vq;
      if constexpr (D == 128) {
      if (a.pend_evict && t0 + 64 >= vq && t0 < vq) {
        // the evicted token vq-1 is in this chunk: its codes and (scale, zero) join the chunk's
        // registers and go to memory (the only reader of those words this launch is here)
        constexpr int PPW = 32 / BITS, VW = 64 * BITS / 32;
        const uint32_t tt = static_cast<uint32_t>(vq - 1 - t0);
        const uint32_t sh = code_shift(BITS, tt % PPW);
        const uint32_t tb = static_cast<uint32_t>(t0 / 64);
#pragma unroll
        for (int hv = 0; hv < 2; ++hv) {
          const uint32_t code = evict_code(er.x[hv], er.mn[hv], er.sc[hv], kLevels) << sh;
#pragma unroll
          for (int qq = 0; qq < VW; ++qq)
            if (qq == (int)(tt / PPW)) {
              cur.w[hv][qq] |= code;
              a.c.vcodes[unit * a.c.geo.vcodes_unit() + ((uint64_t)tb * 128 + lane + 64 * hv) * VW + qq] =
                  cur.w[hv][qq];
            }
          const uint32_t mine = 8 * la + 2 * li;  // the lane's (scale, zero) tokens: mine, mine+1
          if (mine == tt || mine + 1 == tt) {
            if (mine == tt) {
              vp.sz[hv].x = er.sc[hv];
              vp.sz[hv].y = er.mn[hv];
            } else {
              vp.sz[hv].z = er.sc[hv];
              vp.sz[hv].w = er.mn[hv];
            }
            // (G = 32 here: the decode is fused into the launch only for G = 32)
            *reinterpret_cast<float2*>(a.c.vparams + unit * a.c.geo.vparams_unit() +
                                       (((uint64_t)tb * 4 + lc + 2 * hv) * 64 + tt) * 2) =
                make_float2(er.sc[hv], er.mn[hv]);
          }
        }
        if (lane == 0) {
          atomicMax(max_slot(a.c, unit, 0) + kMaxValueScale, __float_as_uint(ev_scale));
          atomicMax(max_slot(a.c, unit, 0) + kMaxValueAbs, __float_as_uint(ev_amax));
        }
      }
      }  // D == 128 (the decode is fused into the launch at head_dim 128 only)
      float w[NRS][8];
#pragma unroll
      for (int rs = 0; rs < NRS; ++rs) {
        const float4* lp = reinterpret_cast<const float4*>(wl + (rs * 4 + li) * ROW + k * 64 + 8 * la);
        const float4 x0 = lp[0], x1 = lp[1];
        const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          w[rs][r] = __builtin_amdgcn_exp2f(fmaf(xs[r], kout, evoff[rs]));  // 2^ev * weight
          lsum[rs] += w[rs][r];
        }
      }
      if (packed) value_operands<NRS, D>(vp, w, A, zacc);
      if constexpr (CPW > 1) {
        const int32_t kn = std::min(chunk_of(std::min(k + 1, nch - 1)), lastv);
        load_value_params<D>(a, unit, kn, la, lc, li, vp);
        load_value_words<BITS, D>(a, unit, kn, lane, next);
      }
      if (packed) value_mfma<BITS, NRS, D>(cur, A, vacc);
      if constexpr (MIXED) {
        if (value_rows) value_fp32<NRS>(a, t0, quarter, la, wl + li * ROW, moff, kout, vfac * kUnit, vrw, vacc);
      }
    };
    if (!EARLY && nch > 0) {
      const int32_t v0 = std::min(chunk_of(0), lastv);
      load_value_params<D>(a, unit, v0, la, lc, li, vp);
      load_value_words<BITS, D>(a, unit, v0, lane, vw0);
    }
    for (int k = 0; k < nch; k += 2) {
      step(k, vw0, vw1);
      if (k + 1 < nch) step(k + 1, vw1, vw0);
    }
  }

  // ---------------- wave partial: reduce l and the zero terms over the 8 blocks
#pragma unroll
  for (int rs = 0; rs < NRS; ++rs) {
    lsum[rs] = sum_over_blocks(lsum[rs]);
#pragma unroll
    for (int hv = 0; hv < HV; ++hv) zacc[rs][hv] = sum_over_blocks(zacc[rs][hv]);
  }
  __syncthreads();  // every wave is done with its logits; reuse LDS for the combine
  float* cw = lds + wave * NH * (D + 2);
#pragma unroll
  for (int rs = 0; rs < NRS; ++rs) {
#pragma unroll
    for (int hv = 0; hv < HV; ++hv) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // zero term of head i, the channel group of channels 32*lc + 64*hv, lives in lane
        // 32*lc + i
        const float z = __shfl(zacc[rs][hv], 32 * lc + i) * vinv;
        cw[(rs * 4 + i) * (D + 2) + lane + 64 * hv] = fmaf(vacc[rs][hv][i], vout, z);
      }
    }
    if (lane < 4) {  // lanes 0..3 hold row li = lane after the reductions
      cw[(rs * 4 + lane) * (D + 2) + D] = nch > 0 ? mrow[rs] : -INFINITY;
      cw[(rs * 4 + lane) * (D + 2) + D + 1] = nch > 0 ? lsum[rs] * vinv : 0.f;
    }
  }
  __syncthreads();
  // the head group's rows hg*NH .. (the unit's heads gq)
  const uint32_t hrows = std::min<uint32_t>(NH, gq - hg * NH);
  float* part = a.ws + (((uint64_t)unit * a.nsplit_total + split_base + split) * gq + hg * NH) * (D + 2);
  if constexpr (EARLY) {
    // wave w writes rows w, w + 4: lane l channels l + 64k, lanes 0 and 1 the row's (m, l),
    // each wave's weight exp2(m_w - M) computed once per row (fewer dependent LDS reads on
    // the critical path of a short launch)
    for (uint32_t h = wave; h < hrows; h += 4) {
      float mw[4], f[4];
      float M = -INFINITY;
#pragma unroll
      for (int wv = 0; wv < 4; ++wv) {
        mw[wv] = lds[wv * NH * (D + 2) + h * (D + 2) + D];
        M = fmaxf(M, mw[wv]);
      }
#pragma unroll
      for (int wv = 0; wv < 4; ++wv) f[wv] = mw[wv] == -INFINITY ? 0.f : exp2f(mw[wv] - M);
#pragma unroll
      for (int k = 0; k < HV; ++k) {
        const uint32_t d = lane + 64 * k;
        float v = 0.f;
#pragma unroll
        for (int wv = 0; wv < 4; ++wv) v += lds[wv * NH * (D + 2) + h * (D + 2) + d] * f[wv];
        part[h * (D + 2) + d] = v;
      }
      if (lane < 2) {
        float v = M;
        if (lane == 1) {
          v = 0.f;
#pragma unroll
          for (int wv = 0; wv < 4; ++wv) v += lds[wv * NH * (D + 2) + h * (D + 2) + D + 1] * f[wv];
        }
        part[h * (D + 2) + D + lane] = v;
      }
    }
  } else {
    for (uint32_t idx = threadIdx.x; idx < hrows * (D + 2); idx += blockDim.x) {
      const uint32_t h = idx / (D + 2), d = idx % (D + 2);
      float M = -INFINITY;
#pragma unroll
      for (int wv = 0; wv < 4; ++wv) M = fmaxf(M, lds[wv * NH * (D + 2) + h * (D + 2) + D]);
      float v = 0.f;
      if (d == D) {
        v = M;
      } else {
#pragma unroll
        for (int wv = 0; wv < 4; ++wv) {
          const float* c = lds + wv * NH * (D + 2) + h * (D + 2);
          const float f = c[D] == -INFINITY ? 0.f : exp2f(c[D] - M);
          v += (d == D + 1 ? c[D + 1] : c[d]) * f;
        }
      }
      part[h * (D + 2) + d] = v;
    }
  }
}

// Chunk launch: workgroups [0, units*nsplit_win) take one window / suffix chunk each (MIXED
// path, started first), the rest a split of 4*kFastCpw packed chunks. Every split writes its
// partial with plain stores; the merge launch that follows on the stream reads them.
//
// Resident workgroups per CU asked of the register allocator per instantiation (4-wave
// workgroups, so also waves per SIMD): it then packs the 4-bit GQA-4 kernel into 128 VGPRs
// (4 waves) and the GQA-8 ones into 168 (3 waves) without spills; head_dim 256 at 4/8 bits
// holds twice the code words and takes two (up to 256 VGPRs).
constexpr int fast_min_groups(int bits, int nrs, int d) {
  return d > 128 ? (bits == 2 ? 3 : 2) : (nrs == 1 && bits <= 4) ? 4 : (bits == 8 && nrs == 2) ? 2 : 3;
}
// SMALL: every wave owns at most one chunk (decode-sized launches): EARLY requests, one
// chunk's logits of LDS; its register use does not set the occupancy of long launches.
template <int BITS, int NRS, int D, bool SMALL = false>
__global__ void __launch_bounds__(kThreads, SMALL ? 2 : fast_min_groups(BITS, NRS, D))
    k_attn_mfma(AttnArgs a) {
  extern __shared__ float lds[];
  // workgroups of (unit, head group) pairs: vu = unit * hgroups + hg. First in the grid, so
  // their latency-bound fp32 rows overlap the packed chunks: at head_dim 128 the window /
  // suffix chunks, at other head_dims the generic splits over the tokens after the packed
  // chunks (one of the two counts is zero).
  const uint32_t nwin = a.units * a.hgroups * a.nsplit_win;
  const uint32_t ngen = a.units * a.nsplit_gen;
  if constexpr (D == 128) {
    if (blockIdx.x < nwin) {
      const uint32_t vu = blockIdx.x / a.nsplit_win;
      mfma_split<BITS, NRS, 1, true, D, SMALL>(a, vu / a.hgroups, blockIdx.x % a.nsplit_win, vu % a.hgroups, lds);
      return;
    }
  } else {
    if (blockIdx.x < ngen) {
      generic_split<BITS, D, 0>(a, blockIdx.x / a.nsplit_gen, blockIdx.x % a.nsplit_gen, lds);
      return;
    }
  }
  const uint32_t blk = blockIdx.x - nwin - ngen, vu = blk / a.nsplit_fast;
  if constexpr (SMALL) {
    mfma_split<BITS, NRS, 1, false, D, true>(a, vu / a.hgroups, blk % a.nsplit_fast, vu % a.hgroups, lds);
  } else {
    mfma_split<BITS, NRS, fast_cpw(BITS, NRS), false, D>(a, vu / a.hgroups, blk % a.nsplit_fast, vu % a.hgroups, lds);
  }
}

// ------------------------------------------------------------------ eight-head 16x16x32 path
// Packed chunks of eight-head units (GQA 5..8, and head groups of 8 above) at head_dim 128,
// G = 32, on v_mfma_f32_16x16x32_f16. Per issue cycle it does four times the multiply-adds of
// the 4x4x4 broadcast form, and vector instructions of other waves issue while it runs (the
// 4x4x4 form holds them off); the decode kernels are bound by the two streams together.
//
// Lane l = 16g + n; D (4 VGPRs) holds rows 4g .. 4g+3 of column n of a 16x16 tile.
// Keys: rows = 16 tokens (tile mt: tokens 16mt .. +15), columns = (head n%8, key group n/8 of
// the chunk), K = 32 channels per K-tile (lane group g: channels 32g + 8kt .. +7), each K-tile
// taken twice into one accumulator, against the hi and then the lo halves of q*scale (B
// operand) with the same eight codes (A operand). A tile's tokens lie in one key group: the
// other group's columns are computed and dropped.
// Values: rows = 16 channels (tile mt: channels 16mt .. +15, value group mt/2), columns =
// (head n%8, parity n/8 of the value group), K = 32 tokens per K-tile (lane group g: tokens
// 16g + 8kt .. +7), hi and lo halves of w*scale as for the keys; the other parity's columns
// are dropped. (Four codes twice in one K-tile against hi-then-lo K slots measured slower:
// the duplicated operand costs a copy per MFMA.)
// A chunk's (scale, zero) pairs are staged in LDS, from which the eight lanes of a head
// column set read them as broadcasts (no cross-lane moves on the vector ALU).
typedef _Float16 h8 __attribute__((ext_vector_type(8)));

constexpr int kWideHeads = 8;     // heads per workgroup (one head group)
// Chunks per wave and workgroups per CU: 2- and 4-bit take 6 chunks and three workgroups per
// CU (the LDS of six chunks' logits, 168 VGPRs); 8-bit, whose code words take more registers,
// 8 chunks and two (up to 256 VGPRs).
constexpr int wide_cpw(int bits) { return bits == 8 ? 8 : 6; }
constexpr int wide_blocks(int bits) { return bits == 8 ? 2 : 3; }
// One chunk's (scale, zero) pairs (512 floats, as stored: keys [group][channel][2], values
// [group][token][2]) are staged in the LDS of the chunk's own logits slot, eight row segments
// of 64 floats: stage float i at row i/64, column 64k + i%64. A key step reads them before it
// writes the slot's logits; a value step writes them after it has read the slot's logits.
// (A separate, bank-padded staging buffer measured no faster and cost a workgroup per CU.)
__device__ __forceinline__ float* wide_stage_at(float* wl, int row, int k, uint32_t i) {
  return wl + (i / 64) * row + k * 64 + (i % 64);
}

__device__ __forceinline__ v4f mfma_wide(h8 a, h8 b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ h8 join(h4 x, h4 y) { return h8{x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]}; }

// One chunk's code words for the lane. Keys: tile mt's token 16mt + n, words BITS*g .. +BITS-1
// of its row (channels 32g .. 32g+31). Values: tile mt's channel 16mt + n, words
// (BITS/2)*g .. of its 64-token block (tokens 16g .. 16g+15).
template <int BITS>
struct WideKeyWords {
  uint32_t w[4][BITS];
};
template <int BITS>
struct WideValueWords {
  uint32_t w[8][BITS / 2];
};

template <int BITS>
__device__ __forceinline__ void wide_load_keys(const AttnArgs& a, uint32_t unit, uint32_t ch, uint32_t g,
                                               uint32_t n, WideKeyWords<BITS>& kw) {
  constexpr int KW = 4 * BITS;  // words per token at head_dim 128
  const uint32_t* base = a.c.kcodes + unit * a.c.geo.kcodes_unit() + ((uint64_t)ch * 64 + n) * KW + BITS * g;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const uint32_t* p = base + 16 * mt * KW;
    if constexpr (BITS == 2) {
      const uint2 x = *reinterpret_cast<const uint2*>(p);
      kw.w[mt][0] = x.x;
      kw.w[mt][1] = x.y;
    } else {
      load_words<BITS>(p, kw.w[mt]);
    }
  }
}
template <int BITS>
__device__ __forceinline__ void wide_load_values(const AttnArgs& a, uint32_t unit, uint32_t tb, uint32_t g,
                                                 uint32_t n, WideValueWords<BITS>& vw) {
  constexpr int VW = 2 * BITS, VG = BITS / 2;  // words per channel per block; the lane's share
  const uint32_t* base = a.c.vcodes + unit * a.c.geo.vcodes_unit() + ((uint64_t)tb * 128 + n) * VW + VG * g;
#pragma unroll
  for (int mt = 0; mt < 8; ++mt) {
    const uint32_t* p = base + 16 * mt * VW;
    if constexpr (VG == 1) {
      vw.w[mt][0] = p[0];
    } else if constexpr (VG == 2) {
      const uint2 x = *reinterpret_cast<const uint2*>(p);
      vw.w[mt][0] = x.x;
      vw.w[mt][1] = x.y;
    } else {
      load_words<VG>(p, vw.w[mt]);
    }
  }
}
// the lane's share of a chunk's (scale, zero) pairs, as stored: keys, group lane/32 of the
// chunk, channels 4*(lane%32) .. +3; values, group lane/16, tokens 4*(lane%16) .. +3
__device__ __forceinline__ void wide_load_key_params(const AttnArgs& a, uint32_t unit, uint32_t ch, uint32_t lane,
                                                     float4& p0, float4& p1) {
  const float4* p = reinterpret_cast<const float4*>(
      a.c.kparams + unit * a.c.geo.kparams_unit() + ((uint64_t)(2 * ch + lane / 32) * 128 + 4 * (lane % 32)) * 2);
  p0 = p[0];
  p1 = p[1];
}
__device__ __forceinline__ void wide_load_value_params(const AttnArgs& a, uint32_t unit, uint32_t tb,
                                                       uint32_t lane, float4& p0, float4& p1) {
  const float4* p = reinterpret_cast<const float4*>(
      a.c.vparams + unit * a.c.geo.vparams_unit() + (((uint64_t)tb * 4 + lane / 16) * 64 + 4 * (lane % 16)) * 2);
  p0 = p[0];
  p1 = p[1];
}
// The lane's eight floats (four (scale, zero) pairs, as loaded) at stage floats 8*lane ..
__device__ __forceinline__ void wide_stage(float* wl, int row, int k, uint32_t lane, float4 p0, float4 p1) {
  float4* s = reinterpret_cast<float4*>(wide_stage_at(wl, row, k, 8 * lane));
  s[0] = p0;
  s[1] = p1;
}

// A operand of tile mt, K-tile kt: the eight codes of the lane's K slots, in element order.
template <int BITS>
__device__ __forceinline__ h8 wide_key_codes(const WideKeyWords<BITS>& kw, int mt, int kt) {
  // channels 32g + 8kt .. +7: 2-bit word 2g + kt/2, elements 8*(kt%2) ..; 4-bit word 4g + kt;
  // 8-bit words 8g + 2kt, +1
  if constexpr (BITS == 2) return join(codes4<2>(kw.w[mt][kt / 2], 2 * (kt % 2)), codes4<2>(kw.w[mt][kt / 2], 2 * (kt % 2) + 1));
  else if constexpr (BITS == 4) return join(codes4<4>(kw.w[mt][kt], 0), codes4<4>(kw.w[mt][kt], 1));
  else return join(codes4<8>(kw.w[mt][2 * kt], 0), codes4<8>(kw.w[mt][2 * kt + 1], 0));
}
template <int BITS>
__device__ __forceinline__ h8 wide_value_codes(const WideValueWords<BITS>& vw, int mt, int kt) {
  // tokens 16g + 8kt .. +7 of the channel: 2-bit word g, elements 8kt ..; 4-bit word 2g + kt;
  // 8-bit words 4g + 2kt, +1
  if constexpr (BITS == 2) return join(codes4<2>(vw.w[mt][0], 2 * kt), codes4<2>(vw.w[mt][0], 2 * kt + 1));
  else if constexpr (BITS == 4) return join(codes4<4>(vw.w[mt][kt], 0), codes4<4>(vw.w[mt][kt], 1));
  else return join(codes4<8>(vw.w[mt][2 * kt], 0), codes4<8>(vw.w[mt][2 * kt + 1], 0));
}

// B operands from eight products: their hi halves and their lo halves (x below 2^15 in
// magnitude)
__device__ __forceinline__ void wide_split8(const float (&x)[8], h8& hi, h8& lo) {
  h4 h0, l0, h1, l1;
  split4(x, h0, l0);
  split4(x + 4, h1, l1);
  hi = join(h0, h1);
  lo = join(l0, l1);
}

// A decode token appended by this launch evicted token vq-1 into the chunk at token t0 (t0 <=
// vq-1 < t0 + 64): the token's codes and (scale, zero) pairs join the wave's registers of the
// chunk (value words vw, the lane's pairs p0 / p1 as wide_load_value_params holds them) and go
// to memory (the only reader of those words in this launch is this wave), and the unit's
// maxima take the row's largest scale and |x|, as the value quantizer would have
// (src/quant.rs:349-375). er is the row in the quantizer's layout (lane holds channels lane and
// 64 + lane, after evict_groups).
template <int BITS>
__device__ __forceinline__ void wide_evict(const AttnArgs& a, uint32_t unit, const EvictRow& er, uint64_t t0,
                                           uint32_t lane, WideValueWords<BITS>& vw, float4& p0, float4& p1,
                                           float ev_scale, float ev_amax) {
  constexpr int PPW = 32 / BITS, VW = 2 * BITS, VG = BITS / 2;
  constexpr float kLevels = static_cast<float>((1 << BITS) - 1);
  const uint32_t g = lane / 16, n = lane % 16;
  const uint32_t tt = static_cast<uint32_t>(a.st.vq - 1 - t0);  // the token within the chunk
  const uint64_t tb = t0 / 64;
  const uint32_t c0 = evict_code(er.x[0], er.mn[0], er.sc[0], kLevels);  // channel lane
  const uint32_t c1 = evict_code(er.x[1], er.mn[1], er.sc[1], kLevels);  // channel 64 + lane
  // lane group tt/16 holds the token's word (tt % 16) / PPW of its share, for channel 16mt + n
  const uint32_t wi = (tt % 16) / PPW, sh = code_shift(BITS, tt % PPW);
#pragma unroll
  for (int mt = 0; mt < 8; ++mt) {
    const uint32_t code = static_cast<uint32_t>(__shfl(static_cast<int>(mt < 4 ? c0 : c1), (16 * mt + n) % 64));
    if (g == tt / 16) {
#pragma unroll
      for (int i = 0; i < VG; ++i) {
        if (i == (int)wi) {
          vw.w[mt][i] |= code << sh;
          a.c.vcodes[unit * a.c.geo.vcodes_unit() + ((uint64_t)tb * 128 + 16 * mt + n) * VW + VG * g + i] = vw.w[mt][i];
        }
      }
    }
  }
  // the pair of group g (channels 32g .. +31: the quantizer's half-wave g % 2 of hv = g / 2) for
  // token tt, held by the lane of group g with n == tt / 4 (pairs of tokens 4n .. 4n + 3)
  float sc = 0.f, mn = 0.f;
#pragma unroll
  for (int cg = 0; cg < 4; ++cg) {
    const float s = lane_value(er.sc[cg / 2], 32 * (cg % 2));
    const float m = lane_value(er.mn[cg / 2], 32 * (cg % 2));
    if (g == (uint32_t)cg) {
      sc = s;
      mn = m;
    }
  }
  if (n == tt / 4) {
    const uint32_t j = tt % 4;
    if (j == 0) {
      p0.x = sc;
      p0.y = mn;
    } else if (j == 1) {
      p0.z = sc;
      p0.w = mn;
    } else if (j == 2) {
      p1.x = sc;
      p1.y = mn;
    } else {
      p1.z = sc;
      p1.w = mn;
    }
    *reinterpret_cast<float2*>(a.c.vparams + unit * a.c.geo.vparams_unit() + (((uint64_t)tb * 4 + g) * 64 + tt) * 2) =
        make_float2(sc, mn);
  }
  if (lane == 0) {
    atomicMax(max_slot(a.c, unit, 0) + kMaxValueScale, __float_as_uint(ev_scale));
    atomicMax(max_slot(a.c, unit, 0) + kMaxValueAbs, __float_as_uint(ev_amax));
  }
}

// EVICT: the launch also appends a decode token whose window eviction lands in the packed
// range (a separate instantiation, so the plain attention keeps its register budget).
template <int BITS, bool EVICT>
__device__ __forceinline__ void wide_split(const AttnArgs& a, uint32_t unit, uint32_t split, uint32_t hg,
                                           float* lds) {
  constexpr int CPW = wide_cpw(BITS), NH = kWideHeads, D = 128;
  constexpr int ROW = CPW * 64 + kRowPad;
  // At 8 bits (two workgroups per CU) a wave raises its issue priority from the start of a
  // chunk step until that step's next-chunk requests are out, so the requests of the SIMD's
  // waves are not held behind the other waves' matrix and vector work (C3 at 8 bits: 68.6 ->
  // 65.0 us). At three workgroups per CU (2 and 4 bits) the same raise cost 40%.
  constexpr bool kRaise = BITS == 8;
  constexpr int kExp = CodeUnit<BITS>::kExp;
  constexpr float kUnit = kExp == 0 ? 1.0f : kExp == -1 ? 0.5f : 0.001953125f;
  const uint32_t b = unit / a.heads, kvh = unit % a.heads;
  const uint32_t lane = threadIdx.x % 64, wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  const uint32_t g = lane / 16, n = lane % 16;
  const uint32_t hq = n % 8;   // head of the lane's column
  const uint32_t sel = n / 8;  // key group of the chunk (keys) / value group parity (values)
  const uint32_t gq = a.gq;
  float* wl = lds + wave * NH * ROW;  // this wave's logits [NH][ROW] (and staging)

  // chunks dealt round-robin over the unit's waves, as in the 4x4x4 path
  const int32_t slots = static_cast<int32_t>(a.nsplit_fast * 4);
  const int32_t slot = static_cast<int32_t>(split * 4 + wave);
  const int32_t span = static_cast<int32_t>(a.chunk_end - a.chunk_begin);
  const int32_t nch = std::min<int32_t>(CPW, std::max<int32_t>(0, (span - slot + slots - 1) / slots));
  // (every owned chunk is packed in keys and values: chunk_end <= min(kq, vq) / 64)
  auto chunk_of = [&](int32_t k) { return static_cast<int32_t>(a.chunk_begin) + slot + k * slots; };

  // one chunk ahead (two ahead measured slower): two buffers of code words; one of (scale,
  // zero) pairs, staged to LDS before the next chunk's are requested into it
  WideKeyWords<BITS> kw0, kw1;
  float4 kp0, kp1;
  if (nch > 0) {
    wide_load_key_params(a, unit, chunk_of(0), lane, kp0, kp1);
    wide_load_keys<BITS>(a, unit, chunk_of(0), g, n, kw0);
  }
  // a decode token appended by this launch evicts token vq-1 from the window: its row, in the
  // value quantizer's layout (channels lane and 64 + lane)
  EvictRow er{};
  if constexpr (EVICT) {
    const float* row = a.c.vring + ((uint64_t)unit * a.c.geo.R + a.pend_vslot) * D;
    er.x[0] = row[lane];
    er.x[1] = row[lane + 64];
  }
  // q in base-2 logit units: head hg*8 + hq, channels 32g .. 32g+31 (0 for padded heads)
  float qv[32];
  float qmax = 0.f;
  {
    const uint32_t h = hg * NH + hq;
    const float s = h < gq ? a.scale2 : 0.f;
    const float* qp = a.query + ((uint64_t)b * a.qh + kvh * gq + min(h, gq - 1)) * D + 32 * g;
#pragma unroll
    for (int r = 0; r < 32; r += 4) {
      const float4 v = *reinterpret_cast<const float4*>(qp + r);
      qv[r] = v.x * s;
      qv[r + 1] = v.y * s;
      qv[r + 2] = v.z * s;
      qv[r + 3] = v.w * s;
    }
#pragma unroll
    for (int r = 0; r < 32; ++r) qmax = fmaxf(qmax, fabsf(qv[r]));
  }
  // power-of-two operand ranges from the unit's largest scales, as in the 4x4x4 path
  qmax = warp_max(qmax);
  float kmax, vmax_all;  // the unit's largest key and value scales
  unit_scale_max(a.c, unit, kmax, vmax_all);
  const int ek = std::min(60, std::max(-100, 15 - __builtin_amdgcn_frexp_expf(qmax * kmax)));
  const float kfac = ldexpf(1.f, ek);
  const float kout = ldexpf(1.f, -ek - kExp);
#pragma unroll
  for (int r = 0; r < 32; ++r) qv[r] *= kfac;

  // ---------------- phase 1: logits of every owned chunk into LDS (scaled by 2^(ek+kExp))
  float mx = -INFINITY;
  {
    auto step = [&](int k, const WideKeyWords<BITS>& cur, WideKeyWords<BITS>& next) {
      if constexpr (kRaise) __builtin_amdgcn_s_setprio(1);
      // this chunk's (scale, zero) pairs to LDS (after the previous chunk's reads of them),
      // then the next chunk's requested (the last step re-reads an L2-resident chunk)
      wide_stage(wl, ROW, k, lane, kp0, kp1);
      const int32_t kn = chunk_of(std::min(k + 1, nch - 1));
      wide_load_key_params(a, unit, kn, lane, kp0, kp1);
      wide_load_keys<BITS>(a, unit, kn, g, n, next);
      if constexpr (kRaise) __builtin_amdgcn_s_setprio(0);
      v4f acc[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) acc[mt] = v4f{0.f, 0.f, 0.f, 0.f};
      float bias = 0.f;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        // channels 32g + 8kt .. +7 of key group sel: four (scale, zero) pairs per float4 pair
        const float4* sp = reinterpret_cast<const float4*>(wide_stage_at(wl, ROW, k, (sel * 128 + 32 * g + 8 * kt) * 2));
        const float4 s[4] = {sp[0], sp[1], sp[2], sp[3]};
        float p[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          p[2 * j] = qv[8 * kt + 2 * j] * s[j].x;
          p[2 * j + 1] = qv[8 * kt + 2 * j + 1] * s[j].z;
          bias = fmaf(qv[8 * kt + 2 * j], s[j].y, bias);
          bias = fmaf(qv[8 * kt + 2 * j + 1], s[j].w, bias);
        }
        h8 bhi, blo;
        wide_split8(p, bhi, blo);
        // two tiles' codes live at a time; each tile's hi and lo products one MFMA apart
#pragma unroll
        for (int m2 = 0; m2 < 4; m2 += 2) {
          const h8 A0 = wide_key_codes<BITS>(cur, m2, kt), A1 = wide_key_codes<BITS>(cur, m2 + 1, kt);
          acc[m2] = mfma_wide(A0, bhi, acc[m2]);
          acc[m2 + 1] = mfma_wide(A1, bhi, acc[m2 + 1]);
          acc[m2] = mfma_wide(A0, blo, acc[m2]);
          acc[m2 + 1] = mfma_wide(A1, blo, acc[m2 + 1]);
        }
      }
      // the zero term of the lane's column over all 128 channels (lane groups g)
      bias += __shfl_xor(bias, 16);
      bias += __shfl_xor(bias, 32);
      const float bu = bias * kUnit;
      // the lane's column is live for the two tiles of its key group: tokens 32*sel + 16*m2 + 4g ..
#pragma unroll
      for (int m2 = 0; m2 < 2; ++m2) {
        const v4f v = sel ? acc[2 + m2] : acc[m2];
        const float4 o = make_float4(v[0] + bu, v[1] + bu, v[2] + bu, v[3] + bu);
        *reinterpret_cast<float4*>(wl + hq * ROW + k * 64 + 32 * sel + 16 * m2 + 4 * g) = o;
        mx = fmaxf(mx, fmaxf(fmaxf(o.x, o.y), fmaxf(o.z, o.w)));
      }
    };
    for (int k = 0; k < nch; k += 2) {
      step(k, kw0, kw1);
      if (k + 1 < nch) step(k + 1, kw1, kw0);
    }
  }
  // wave max per head: the lanes of head hq (both key groups, four lane groups)
  mx = fmaxf(mx, __shfl_xor(mx, 8));
  mx = fmaxf(mx, __shfl_xor(mx, 16));
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  const float mrow = mx * kout;

  // the value operands' range: the unit's largest value scale, raised by the evicted row's (as
  // the append would have raised it)
  float vmax = vmax_all;
  float ev_scale = 0.f, ev_amax = 0.f;
  if constexpr (EVICT) {
    evict_groups(er, static_cast<float>((1 << BITS) - 1), ev_scale, ev_amax);
    vmax = fmaxf(vmax, ev_scale);
  }
  const int ev = std::min(60, std::max(-100, 15 - __builtin_amdgcn_frexp_expf(vmax)));
  const float vout = ldexpf(1.f, -ev - kExp);
  const float moff = mrow == -INFINITY ? 0.f : mrow;
  const float evoff = static_cast<float>(ev) - moff;  // weights times 2^ev from the exponential
  const float vinv = ldexpf(1.f, -ev);

  // ---------------- phase 2: value mix
  v4f vacc[8];
#pragma unroll
  for (int mt = 0; mt < 8; ++mt) vacc[mt] = v4f{0.f, 0.f, 0.f, 0.f};
  float zacc[2] = {0.f, 0.f};  // zero terms of value groups sel, 2 + sel
  float lsum = 0.f;
  {
    WideValueWords<BITS> vw0, vw1;
    float4 vp0, vp1;
    if (nch > 0) {
      wide_load_value_params(a, unit, chunk_of(0), lane, vp0, vp1);
      wide_load_values<BITS>(a, unit, chunk_of(0), g, n, vw0);
    }
    auto step = [&](int k, WideValueWords<BITS>& cur, WideValueWords<BITS>& next) {
      if constexpr (kRaise) __builtin_amdgcn_s_setprio(1);
      // weights (times 2^ev) of head hq, tokens 16g .. 16g+15, read from the slot before the
      // chunk's (scale, zero) pairs are staged over it
      float4 lg[4];
      {
        const float4* lp = reinterpret_cast<const float4*>(wl + hq * ROW + k * 64 + 16 * g);
#pragma unroll
        for (int r = 0; r < 4; ++r) lg[r] = lp[r];
      }
      if constexpr (EVICT) {
        const uint64_t t0 = (uint64_t)chunk_of(k) * 64;
        if (t0 < a.st.vq && t0 + 64 >= a.st.vq) wide_evict<BITS>(a, unit, er, t0, lane, cur, vp0, vp1, ev_scale, ev_amax);
      }
      wide_stage(wl, ROW, k, lane, vp0, vp1);
      const int32_t kn = chunk_of(std::min(k + 1, nch - 1));
      wide_load_value_params(a, unit, kn, lane, vp0, vp1);
      wide_load_values<BITS>(a, unit, kn, g, n, next);
      if constexpr (kRaise) __builtin_amdgcn_s_setprio(0);
      float w[16];
      {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float4 x = lg[r];
          w[4 * r] = __builtin_amdgcn_exp2f(fmaf(x.x, kout, evoff));
          w[4 * r + 1] = __builtin_amdgcn_exp2f(fmaf(x.y, kout, evoff));
          w[4 * r + 2] = __builtin_amdgcn_exp2f(fmaf(x.z, kout, evoff));
          w[4 * r + 3] = __builtin_amdgcn_exp2f(fmaf(x.w, kout, evoff));
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) lsum += w[r];
      }
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
        for (int pr = 0; pr < 2; ++pr) {

          // value group 2*pr + sel, tokens 16g + 8kt .. +7
          const float4* sp =
              reinterpret_cast<const float4*>(wide_stage_at(wl, ROW, k, ((2 * pr + sel) * 64 + 16 * g + 8 * kt) * 2));
          const float4 s[4] = {sp[0], sp[1], sp[2], sp[3]};
          float p[8];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            p[2 * j] = w[8 * kt + 2 * j] * s[j].x;
            p[2 * j + 1] = w[8 * kt + 2 * j + 1] * s[j].z;
            zacc[pr] = fmaf(w[8 * kt + 2 * j], s[j].y, zacc[pr]);
            zacc[pr] = fmaf(w[8 * kt + 2 * j + 1], s[j].w, zacc[pr]);
          }
          h8 bhi, blo;
          wide_split8(p, bhi, blo);
#pragma unroll
          for (int m2 = 0; m2 < 4; m2 += 2) {
            const int t0 = 4 * pr + m2;
            const h8 A0 = wide_value_codes<BITS>(cur, t0, kt), A1 = wide_value_codes<BITS>(cur, t0 + 1, kt);
            vacc[t0] = mfma_wide(A0, bhi, vacc[t0]);
            vacc[t0 + 1] = mfma_wide(A1, bhi, vacc[t0 + 1]);
            vacc[t0] = mfma_wide(A0, blo, vacc[t0]);
            vacc[t0 + 1] = mfma_wide(A1, blo, vacc[t0 + 1]);
          }
        }
      }
    };
    for (int k = 0; k < nch; k += 2) {
      step(k, vw0, vw1);
      if (k + 1 < nch) step(k + 1, vw1, vw0);
    }
  }

  // ---------------- wave partial: sums over the lane groups, then the output rows
  lsum += __shfl_xor(lsum, 16);
  lsum += __shfl_xor(lsum, 32);
#pragma unroll
  for (int pr = 0; pr < 2; ++pr) {
    zacc[pr] += __shfl_xor(zacc[pr], 16);
    zacc[pr] += __shfl_xor(zacc[pr], 32);
  }
  __syncthreads();  // every wave is done with its logits; reuse LDS for the combine
  float* cw = lds + wave * NH * (D + 2);
  // the lane's column is live for the tiles of parity sel: tiles 4*pr + 2*sel + m2, channels
  // 16 * tile + 4g .. +3
#pragma unroll
  for (int pr = 0; pr < 2; ++pr) {
    const float z = zacc[pr] * vinv;
#pragma unroll
    for (int m2 = 0; m2 < 2; ++m2) {
      const v4f v = sel ? vacc[4 * pr + 2 + m2] : vacc[4 * pr + m2];
      const uint32_t c0 = 16 * (4 * pr + 2 * sel + m2) + 4 * g;
      float2* o = reinterpret_cast<float2*>(cw + hq * (D + 2) + c0);
      o[0] = make_float2(fmaf(v[0], vout, z), fmaf(v[1], vout, z));
      o[1] = make_float2(fmaf(v[2], vout, z), fmaf(v[3], vout, z));
    }
  }
  if (g == 0 && sel == 0) {
    cw[hq * (D + 2) + D] = nch > 0 ? mrow : -INFINITY;
    cw[hq * (D + 2) + D + 1] = nch > 0 ? lsum * vinv : 0.f;
  }
  __syncthreads();
  const uint32_t hrows = std::min<uint32_t>(NH, gq - hg * NH);
  float* part = a.ws + (((uint64_t)unit * a.nsplit_total + split) * gq + hg * NH) * (D + 2);
  for (uint32_t idx = threadIdx.x; idx < hrows * (D + 2); idx += blockDim.x) {
    const uint32_t h = idx / (D + 2), d = idx % (D + 2);
    float M = -INFINITY;
#pragma unroll
    for (int wv = 0; wv < 4; ++wv) M = fmaxf(M, lds[wv * NH * (D + 2) + h * (D + 2) + D]);
    float v = 0.f;
    if (d == D) {
      v = M;
    } else {
#pragma unroll
      for (int wv = 0; wv < 4; ++wv) {
        const float* c = lds + wv * NH * (D + 2) + h * (D + 2);
        const float f = c[D] == -INFINITY ? 0.f : exp2f(c[D] - M);
        v += (d == D + 1 ? c[D + 1] : c[d]) * f;
      }
    }
    part[h * (D + 2) + d] = v;
  }
}

// Eight-head launch at head_dim 128, G = 32: the window / suffix chunk workgroups first (the
// 4x4x4 MIXED path), then the packed splits on the 16x16x32 path, wide_blocks(BITS)
// workgroups per CU. Requests two chunks ahead measured slower than one. A launch that also
// appends a decode token (EVICT) takes the register budget of two workgroups per CU, so the
// eviction's registers spill nothing (a decode launch is latency-bound).
template <int BITS, bool EVICT>
__global__ void __launch_bounds__(kThreads, EVICT ? 2 : wide_blocks(BITS)) k_attn_wide(AttnArgs a) {
  extern __shared__ float lds[];
  const uint32_t nwin = a.units * a.hgroups * a.nsplit_win;
  if (blockIdx.x < nwin) {
    const uint32_t vu = blockIdx.x / a.nsplit_win;
    mfma_split<BITS, 2, 1, true, 128>(a, vu / a.hgroups, blockIdx.x % a.nsplit_win, vu % a.hgroups, lds);
    return;
  }
  const uint32_t blk = blockIdx.x - nwin, vu = blk / a.nsplit_fast;
  wide_split<BITS, EVICT>(a, vu / a.hgroups, blk % a.nsplit_fast, vu % a.hgroups, lds);
}

// ------------------------------------------------------------------ sixteen-head 16x16x32 path
// GQA 16 (or a multiple of 16) at head_dim 128, G = 32: the MFMA's 16 columns are the 16 heads
// of a head group, so the two key groups of a chunk (and its four value groups) take B
// operands of their own and no column is spent on another group's scales. Each chunk is read
// once for the 16 heads; the eight-head form reads it once per eight. Layout and chunk
// dealing as in wide_split: lane (g, n) holds column n (head 16*hg + n) and K slots 8g .. 8g+7.
constexpr int kWide16Heads = 16;
constexpr int kWide16Cpw = 4;     // chunks per wave: four chunks of 16 heads' logits, 16.6 KB
constexpr int kWide16Blocks = 2;  // workgroups per CU (66.6 KB of LDS each)

template <int BITS>
__device__ __forceinline__ void wide16_split(const AttnArgs& a, uint32_t unit, uint32_t split, uint32_t hg,
                                             float* lds) {
  constexpr int CPW = kWide16Cpw, NH = kWide16Heads, D = 128;
  constexpr int ROW = CPW * 64 + kRowPad;
  // At 2 bits a wave raises its issue priority from the start of a chunk step until that
  // step's next-chunk requests are out, as the eight-head kernel does at 8 bits (GQA 16 at
  // batch 4: 35.3 -> 33.7 us; 128 q / 8 KV heads at batch 16: 198.5 -> 194.0 us). At 4 bits
  // it made no difference and at 8 bits it cost 25%.
  constexpr bool kRaise = BITS == 2;
  constexpr int kExp = CodeUnit<BITS>::kExp;
  constexpr float kUnit = kExp == 0 ? 1.0f : kExp == -1 ? 0.5f : 0.001953125f;
  const uint32_t b = unit / a.heads, kvh = unit % a.heads;
  const uint32_t lane = threadIdx.x % 64, wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  const uint32_t g = lane / 16, n = lane % 16;  // n: the lane's column (head)
  const uint32_t gq = a.gq;
  float* wl = lds + wave * NH * ROW;  // this wave's logits [NH][ROW] (and staging)

  const int32_t slots = static_cast<int32_t>(a.nsplit_fast * 4);
  const int32_t slot = static_cast<int32_t>(split * 4 + wave);
  const int32_t span = static_cast<int32_t>(a.chunk_end - a.chunk_begin);
  const int32_t nch = std::min<int32_t>(CPW, std::max<int32_t>(0, (span - slot + slots - 1) / slots));
  auto chunk_of = [&](int32_t k) { return static_cast<int32_t>(a.chunk_begin) + slot + k * slots; };

  WideKeyWords<BITS> kw0, kw1;
  float4 kp0, kp1;
  if (nch > 0) {
    wide_load_key_params(a, unit, chunk_of(0), lane, kp0, kp1);
    wide_load_keys<BITS>(a, unit, chunk_of(0), g, n, kw0);
  }
  // q in base-2 logit units: head hg*16 + n, channels 32g .. 32g+31 (0 for padded heads)
  float qv[32];
  float qmax = 0.f;
  {
    const uint32_t h = hg * NH + n;
    const float s = h < gq ? a.scale2 : 0.f;
    const float* qp = a.query + ((uint64_t)b * a.qh + kvh * gq + min(h, gq - 1)) * D + 32 * g;
#pragma unroll
    for (int r = 0; r < 32; r += 4) {
      const float4 v = *reinterpret_cast<const float4*>(qp + r);
      qv[r] = v.x * s;
      qv[r + 1] = v.y * s;
      qv[r + 2] = v.z * s;
      qv[r + 3] = v.w * s;
    }
#pragma unroll
    for (int r = 0; r < 32; ++r) qmax = fmaxf(qmax, fabsf(qv[r]));
  }
  qmax = warp_max(qmax);
  float kmax, vmax_all;  // the unit's largest key and value scales
  unit_scale_max(a.c, unit, kmax, vmax_all);
  const int ek = std::min(60, std::max(-100, 15 - __builtin_amdgcn_frexp_expf(qmax * kmax)));
  const float kfac = ldexpf(1.f, ek);
  const float kout = ldexpf(1.f, -ek - kExp);
#pragma unroll
  for (int r = 0; r < 32; ++r) qv[r] *= kfac;

  // ---------------- phase 1: logits of every owned chunk into LDS (scaled by 2^(ek+kExp))
  float mx = -INFINITY;
  {
    auto step = [&](int k, const WideKeyWords<BITS>& cur, WideKeyWords<BITS>& next) {
      if constexpr (kRaise) __builtin_amdgcn_s_setprio(1);
      wide_stage(wl, ROW, k, lane, kp0, kp1);
      const int32_t kn = chunk_of(std::min(k + 1, nch - 1));
      wide_load_key_params(a, unit, kn, lane, kp0, kp1);
      wide_load_keys<BITS>(a, unit, kn, g, n, next);
      if constexpr (kRaise) __builtin_amdgcn_s_setprio(0);
      v4f acc[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) acc[mt] = v4f{0.f, 0.f, 0.f, 0.f};
      float bias[2] = {0.f, 0.f};
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        // channels 32g + 8kt .. +7: one B per key group (tiles 0, 1 take group 0; 2, 3 group 1)
        h8 bhi[2], blo[2];
#pragma unroll
        for (int grp = 0; grp < 2; ++grp) {
          const float4* sp = reinterpret_cast<const float4*>(wide_stage_at(wl, ROW, k, (grp * 128 + 32 * g + 8 * kt) * 2));
          const float4 sv[4] = {sp[0], sp[1], sp[2], sp[3]};
          float p[8];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            p[2 * j] = qv[8 * kt + 2 * j] * sv[j].x;
            p[2 * j + 1] = qv[8 * kt + 2 * j + 1] * sv[j].z;
            bias[grp] = fmaf(qv[8 * kt + 2 * j], sv[j].y, bias[grp]);
            bias[grp] = fmaf(qv[8 * kt + 2 * j + 1], sv[j].w, bias[grp]);
          }
          wide_split8(p, bhi[grp], blo[grp]);
        }
#pragma unroll
        for (int m2 = 0; m2 < 4; m2 += 2) {
          const h8 A0 = wide_key_codes<BITS>(cur, m2, kt), A1 = wide_key_codes<BITS>(cur, m2 + 1, kt);
          acc[m2] = mfma_wide(A0, bhi[m2 / 2], acc[m2]);
          acc[m2 + 1] = mfma_wide(A1, bhi[m2 / 2], acc[m2 + 1]);
          acc[m2] = mfma_wide(A0, blo[m2 / 2], acc[m2]);
          acc[m2 + 1] = mfma_wide(A1, blo[m2 / 2], acc[m2 + 1]);
        }
      }
      // each key group's zero term of the lane's column over all 128 channels (lane groups g)
#pragma unroll
      for (int grp = 0; grp < 2; ++grp) {
        bias[grp] += __shfl_xor(bias[grp], 16);
        bias[grp] += __shfl_xor(bias[grp], 32);
      }
      // tile mt: tokens 16mt + 4g .. +3 of key group mt / 2
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const float bu = bias[mt / 2] * kUnit;
        const v4f v = acc[mt];
        const float4 o = make_float4(v[0] + bu, v[1] + bu, v[2] + bu, v[3] + bu);
        *reinterpret_cast<float4*>(wl + n * ROW + k * 64 + 16 * mt + 4 * g) = o;
        mx = fmaxf(mx, fmaxf(fmaxf(o.x, o.y), fmaxf(o.z, o.w)));
      }
    };
    for (int k = 0; k < nch; k += 2) {
      step(k, kw0, kw1);
      if (k + 1 < nch) step(k + 1, kw1, kw0);
    }
  }
  // wave max per head: the four lane groups of column n
  mx = fmaxf(mx, __shfl_xor(mx, 16));
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  const float mrow = mx * kout;

  const float vmax = vmax_all;
  const int ev = std::min(60, std::max(-100, 15 - __builtin_amdgcn_frexp_expf(vmax)));
  const float vout = ldexpf(1.f, -ev - kExp);
  const float moff = mrow == -INFINITY ? 0.f : mrow;
  const float evoff = static_cast<float>(ev) - moff;  // weights times 2^ev from the exponential
  const float vinv = ldexpf(1.f, -ev);

  // ---------------- phase 2: value mix
  v4f vacc[8];
#pragma unroll
  for (int mt = 0; mt < 8; ++mt) vacc[mt] = v4f{0.f, 0.f, 0.f, 0.f};
  float zacc[4] = {0.f, 0.f, 0.f, 0.f};  // zero terms of the four value groups
  float lsum = 0.f;
  {
    WideValueWords<BITS> vw0, vw1;
    float4 vp0, vp1;
    if (nch > 0) {
      wide_load_value_params(a, unit, chunk_of(0), lane, vp0, vp1);
      wide_load_values<BITS>(a, unit, chunk_of(0), g, n, vw0);
    }
    auto step = [&](int k, const WideValueWords<BITS>& cur, WideValueWords<BITS>& next) {
      if constexpr (kRaise) __builtin_amdgcn_s_setprio(1);
      // weights (times 2^ev) of head n, tokens 16g .. 16g+15, read from the slot before the
      // chunk's (scale, zero) pairs are staged over it
      float4 lg[4];
      {
        const float4* lp = reinterpret_cast<const float4*>(wl + n * ROW + k * 64 + 16 * g);
#pragma unroll
        for (int r = 0; r < 4; ++r) lg[r] = lp[r];
      }
      wide_stage(wl, ROW, k, lane, vp0, vp1);
      const int32_t kn = chunk_of(std::min(k + 1, nch - 1));
      wide_load_value_params(a, unit, kn, lane, vp0, vp1);
      wide_load_values<BITS>(a, unit, kn, g, n, next);
      if constexpr (kRaise) __builtin_amdgcn_s_setprio(0);
      float w[16];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float4 x = lg[r];
        w[4 * r] = __builtin_amdgcn_exp2f(fmaf(x.x, kout, evoff));
        w[4 * r + 1] = __builtin_amdgcn_exp2f(fmaf(x.y, kout, evoff));
        w[4 * r + 2] = __builtin_amdgcn_exp2f(fmaf(x.z, kout, evoff));
        w[4 * r + 3] = __builtin_amdgcn_exp2f(fmaf(x.w, kout, evoff));
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) lsum += w[r];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
        for (int cg = 0; cg < 4; ++cg) {
          // value group cg (channel tiles 2cg, 2cg+1), tokens 16g + 8kt .. +7
          const float4* sp = reinterpret_cast<const float4*>(wide_stage_at(wl, ROW, k, (cg * 64 + 16 * g + 8 * kt) * 2));
          const float4 sv[4] = {sp[0], sp[1], sp[2], sp[3]};
          float p[8];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            p[2 * j] = w[8 * kt + 2 * j] * sv[j].x;
            p[2 * j + 1] = w[8 * kt + 2 * j + 1] * sv[j].z;
            zacc[cg] = fmaf(w[8 * kt + 2 * j], sv[j].y, zacc[cg]);
            zacc[cg] = fmaf(w[8 * kt + 2 * j + 1], sv[j].w, zacc[cg]);
          }
          h8 bhi, blo;
          wide_split8(p, bhi, blo);
          const h8 A0 = wide_value_codes<BITS>(cur, 2 * cg, kt), A1 = wide_value_codes<BITS>(cur, 2 * cg + 1, kt);
          vacc[2 * cg] = mfma_wide(A0, bhi, vacc[2 * cg]);
          vacc[2 * cg + 1] = mfma_wide(A1, bhi, vacc[2 * cg + 1]);
          vacc[2 * cg] = mfma_wide(A0, blo, vacc[2 * cg]);
          vacc[2 * cg + 1] = mfma_wide(A1, blo, vacc[2 * cg + 1]);
        }
      }
    };
    for (int k = 0; k < nch; k += 2) {
      step(k, vw0, vw1);
      if (k + 1 < nch) step(k + 1, vw1, vw0);
    }
  }

  // ---------------- wave partial: sums over the lane groups, then the output rows
  lsum += __shfl_xor(lsum, 16);
  lsum += __shfl_xor(lsum, 32);
#pragma unroll
  for (int cg = 0; cg < 4; ++cg) {
    zacc[cg] += __shfl_xor(zacc[cg], 16);
    zacc[cg] += __shfl_xor(zacc[cg], 32);
  }
  __syncthreads();  // every wave is done with its logits; reuse LDS for the combine
  float* cw = lds + wave * NH * (D + 2);
  // tile mt: channels 16mt + 4g .. +3 of head n (value group mt / 2)
#pragma unroll
  for (int mt = 0; mt < 8; ++mt) {
    const float z = zacc[mt / 2] * vinv;
    const v4f v = vacc[mt];
    float2* o = reinterpret_cast<float2*>(cw + n * (D + 2) + 16 * mt + 4 * g);
    o[0] = make_float2(fmaf(v[0], vout, z), fmaf(v[1], vout, z));
    o[1] = make_float2(fmaf(v[2], vout, z), fmaf(v[3], vout, z));
  }
  if (g == 0) {
    cw[n * (D + 2) + D] = nch > 0 ? mrow : -INFINITY;
    cw[n * (D + 2) + D + 1] = nch > 0 ? lsum * vinv : 0.f;
  }
  __syncthreads();
  const uint32_t hrows = std::min<uint32_t>(NH, gq - hg * NH);
  float* part = a.ws + (((uint64_t)unit * a.nsplit_total + split) * gq + hg * NH) * (D + 2);
  for (uint32_t idx = threadIdx.x; idx < hrows * (D + 2); idx += blockDim.x) {
    const uint32_t h = idx / (D + 2), d = idx % (D + 2);
    float M = -INFINITY;
#pragma unroll
    for (int wv = 0; wv < 4; ++wv) M = fmaxf(M, lds[wv * NH * (D + 2) + h * (D + 2) + D]);
    float v = 0.f;
    if (d == D) {
      v = M;
    } else {
#pragma unroll
      for (int wv = 0; wv < 4; ++wv) {
        const float* c = lds + wv * NH * (D + 2) + h * (D + 2);
        const float f = c[D] == -INFINITY ? 0.f : exp2f(c[D] - M);
        v += (d == D + 1 ? c[D + 1] : c[d]) * f;
      }
    }
    part[h * (D + 2) + d] = v;
  }
}

// Sixteen-head launch at head_dim 128, G = 32, GQA a multiple of 16: the window / suffix chunk
// workgroups first (the 4x4x4 MIXED path, in head groups of eight), then the packed splits on
// the sixteen-head 16x16x32 path (head groups of sixteen), two workgroups per CU.
template <int BITS>
__global__ void __launch_bounds__(kThreads, kWide16Blocks) k_attn_wide16(AttnArgs a) {
  extern __shared__ float lds[];
  const uint32_t nwin = a.units * a.hgroups * a.nsplit_win;
  if (blockIdx.x < nwin) {
    const uint32_t vu = blockIdx.x / a.nsplit_win;
    mfma_split<BITS, 2, 1, true, 128>(a, vu / a.hgroups, blockIdx.x % a.nsplit_win, vu % a.hgroups, lds);
    return;
  }
  const uint32_t blk = blockIdx.x - nwin, vu = blk / a.nsplit_fast;
  wide16_split<BITS>(a, vu / a.hgroups_fast, blk % a.nsplit_fast, vu % a.hgroups_fast, lds);
}

// Arguments of session s of a batched call: its queries, partials and suffix.
__device__ __forceinline__ AttnArgs session_args(const AttnArgs& a, const SessionTable& t,
                                                 uint32_t s) {
  AttnArgs as = a;
  const SessionDesc d = t.d[s];
  as.query = a.query + s * a.q_sess_stride;
  as.ws = a.ws + s * a.ws_sess_stride;
  as.suffix_k = d.k;
  as.suffix_v = d.v;
  as.L = d.len;
  as.suffix_stride = d.stride;
  as.total = a.seq + d.len;
  as.win_end = static_cast<uint32_t>((as.total + 63) / 64);
  return as;
}

// Packed chunks per wave in a batched-sessions launch: a workgroup's chunks (4*kSessCpw*8 KB at
// 2-bit) are re-read for every session, so they are kept few enough to stay cache resident.
constexpr int kSessCpw = 4;

// Batched sessions over one prefix: workgroups [0, nsess*units*nsplit_win) take one window /
// suffix chunk of one session; the rest one packed-chunk split of a unit, for every session
// in turn (the split's chunks are re-read from L2, not HBM, after the first session).
template <int BITS, int NRS>
__global__ void __launch_bounds__(kThreads, BITS == 2 && NRS == 1 ? 3 : 2) k_attn_sessions(AttnArgs a, SessionTable t) {
  extern __shared__ float lds[];
  const uint32_t per_sess = a.units * a.nsplit_win;
  const uint32_t nwin = a.nsess * per_sess;
  if (blockIdx.x < nwin) {
    const uint32_t s = blockIdx.x / per_sess, r = blockIdx.x % per_sess;
    const AttnArgs as = session_args(a, t, s);
    mfma_split<BITS, NRS, 1, true, 128>(as, r / a.nsplit_win, r % a.nsplit_win, 0, lds);
  } else {
    const uint32_t blk = blockIdx.x - nwin;
    const uint32_t unit = blk / a.nsplit_fast, split = blk % a.nsplit_fast;
    for (uint32_t s = 0; s < a.nsess; ++s) {
      AttnArgs as = a;
      as.query = a.query + s * a.q_sess_stride;
      as.ws = a.ws + s * a.ws_sess_stride;
      mfma_split<BITS, NRS, kSessCpw, false, 128>(as, unit, split, 0, lds);
      __syncthreads();  // the next session reuses the LDS
    }
  }
}

// Session suffixes of the shared-prefix form (fp32 rows, head_dim 128, GQA <= 8): one
// workgroup per (session, unit, run of kSufTokens suffix tokens) writes one partial per head
// into split nsplit_fast + run (runs past a session's suffix write empty partials). Keys:
// quad l/4 of wave w owns tokens 32w + l/4 and 32w + 16 + l/4, 32 channels per lane, its dot
// products summed across the quad; values: half-wave h of wave w owns rows 32w + 2j + h
// (j < 16), lane l channels 4 (l % 32) .. + 3, and the eight half-waves' sums meet in LDS.
// Every load of a workgroup is issued before the first wait.
// Raw buffer resource over `floats` floats at p (stride 0, 32-bit data format): loads at byte
// offsets past the range return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const float* p, uint32_t floats) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), 0, static_cast<int>(floats * 4), 0x00020000);
}
__device__ __forceinline__ float4 rsrc_load4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  using u4 = uint32_t __attribute__((ext_vector_type(4)));
  const u4 x = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0);
  return make_float4(__uint_as_float(x.x), __uint_as_float(x.y), __uint_as_float(x.z), __uint_as_float(x.w));
}
__device__ __forceinline__ float2 rsrc_load2(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  using u2 = uint32_t __attribute__((ext_vector_type(2)));
  const u2 x = __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, 0);
  return make_float2(__uint_as_float(x.x), __uint_as_float(x.y));
}

constexpr uint32_t kSufTokens = 128;
constexpr uint32_t kSufMaxHeads = 8;
constexpr uint32_t kSufMergeRound = 16;  // GEMM split partials a wave loads per round

// Output row (sess, unit, h) of the shared-prefix form: the GEMM splits' partials [0,
// nsplit_fast) merged by log-sum-exp with the suffix partial (m, l, o) the wave holds (lane l:
// channels 2l, 2l + 1), in rounds of kSufMergeRound independent loads; the (m, l) pairs are
// wave-uniform.
__device__ __forceinline__ void merge_suffix_row(const AttnArgs& a, uint32_t sess, uint32_t unit, uint32_t h,
                                                 uint32_t lane, float m, float l, float2 o) {
  constexpr uint32_t D = 128, RB = kSufMergeRound;
  const uint32_t gq = a.gq, ns = a.nsplit_fast;
  const uint64_t stride = (uint64_t)gq * (D + 2);
  const float* base = a.ws + (uint64_t)sess * a.ws_sess_stride + ((uint64_t)unit * a.nsplit_total * gq + h) * (D + 2);
  for (uint32_t s0 = 0; s0 < ns; s0 += RB) {
    float2 v[RB];
    float ms[RB], ls[RB];
#pragma unroll
    for (uint32_t j = 0; j < RB; ++j) {
      const float* ps = base + (uint64_t)std::min(s0 + j, ns - 1) * stride;
      ms[j] = s0 + j < ns ? ps[D] : -INFINITY;
      ls[j] = ps[D + 1];
      v[j] = *reinterpret_cast<const float2*>(ps + 2 * lane);
    }
    float bm = m;
#pragma unroll
    for (uint32_t j = 0; j < RB; ++j) bm = fmaxf(bm, ms[j]);
    if (bm != -INFINITY) {
      const float r = __builtin_amdgcn_exp2f(m - bm);  // 0 while m is -inf
      l *= r;
      o.x *= r;
      o.y *= r;
#pragma unroll
      for (uint32_t j = 0; j < RB; ++j) {
        const float f = ms[j] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ms[j] - bm);
        l = fmaf(ls[j], f, l);
        o.x = fmaf(v[j].x, f, o.x);
        o.y = fmaf(v[j].y, f, o.y);
      }
      m = bm;
    }
  }
  const uint32_t b = unit / a.heads, kvh = unit % a.heads;
  float* out = a.out + (uint64_t)sess * a.q_sess_stride + ((uint64_t)b * a.qh + kvh * gq + h) * D;
  *reinterpret_cast<float2*>(out + 2 * lane) = make_float2(o.x / l, o.y / l);
}

// MERGED (a launch group whose suffixes fit one run, after k_attn_shared): one workgroup per
// (session, unit) computes its suffix partial and merges it with the GEMM splits' partials
// into the output (merge_suffix_row), in place of writing a partial for k_attn_merge.
template <bool MERGED>
__global__ void __launch_bounds__(kThreads) k_attn_suffix(AttnArgs a, SessionTable t) {
  constexpr uint32_t D = 128;
  __shared__ float qs[kSufMaxHeads][D];
  __shared__ float sp[kSufMaxHeads][kSufTokens];
  __shared__ float ml[kSufMaxHeads][2];
  __shared__ float red[4][2][kSufMaxHeads][D];  // [wave][half-wave][head][channel]
  const uint32_t lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  const uint32_t gq = a.gq;
  const uint32_t runs = MERGED ? 1u : a.nsplit_win;
  const uint32_t per_sess = a.units * runs;
  const uint32_t sess = blockIdx.x / per_sess, rem = blockIdx.x % per_sess;
  const uint32_t unit = rem / runs, run = rem % runs;
  const SessionDesc d = t.d[sess];
  const uint64_t t0 = (uint64_t)run * kSufTokens;
  const uint32_t n = d.len > t0 ? static_cast<uint32_t>(std::min<uint64_t>(kSufTokens, d.len - t0)) : 0u;
  const uint32_t b = unit / a.heads, kvh = unit % a.heads;
  if (n == 0) {
    if constexpr (MERGED) {
      for (uint32_t h = wave; h < gq; h += 4) merge_suffix_row(a, sess, unit, h, lane, -INFINITY, 0.f, make_float2(0.f, 0.f));
      return;
    }
    // no token of this session in the run (its suffix arrays may be absent): empty partials
    for (uint32_t h = wave; h < gq; h += 4) {
      float* part = a.ws + (uint64_t)sess * a.ws_sess_stride +
                    (((uint64_t)unit * a.nsplit_total + a.nsplit_fast + run) * gq + h) * (D + 2);
      *reinterpret_cast<float2*>(part + 2 * lane) = make_float2(0.f, 0.f);
      if (lane == 0) {
        part[D] = -INFINITY;
        part[D + 1] = 0.f;
      }
    }
    return;
  }
  // Loads in the order they are used, all issued before the first wait: the queries (four
  // floats per thread: gq * D <= 4 * kThreads), this wave's keys (half a row per lane), its
  // values (two channels per lane). The dot products then start as the keys arrive, while the
  // values are still on their way.
  static_assert(kSufMaxHeads * D == 4 * kThreads, "one float4 of queries per thread");
  const float* qp = a.query + (uint64_t)sess * a.q_sess_stride + ((uint64_t)b * a.qh + kvh * gq) * D;
  const bool qlive = 4 * threadIdx.x < gq * D;
  const float4 q4 = reinterpret_cast<const float4*>(qp)[qlive ? threadIdx.x : 0];
  __builtin_amdgcn_sched_barrier(0);
  // The run's rows through buffer resources of n rows: a row past n reads as zeros (its weight
  // is 0) without a memory request and without a branch around the load.
  // Keys: quad q = l / 4 of wave w owns rows 32w + q (pass 0) and 32w + 16 + q (pass 1); lane
  // k = l % 4 of the quad holds channels 16i + 4k .. + 3 (i < 8), so each load instruction
  // reads 64 contiguous bytes of 16 rows.
  const uint32_t hh = lane / 32, qd4 = lane / 4, kq = lane % 4;
  const __amdgpu_buffer_rsrc_t krs = rows_rsrc(d.k + unit * d.stride + t0 * D, n * D);
  float4 kv[16];
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int i = 0; i < 8; ++i)
      kv[8 * p + i] = rsrc_load4(krs, ((32 * wave + 16 * p + qd4) * D + 16 * i + 4 * kq) * 4);
  __builtin_amdgcn_sched_barrier(0);
  const __amdgpu_buffer_rsrc_t vrs = rows_rsrc(d.v + unit * d.stride + t0 * D, n * D);
  float4 vv[16];  // row 32w + 2j + hh, channels 4 (l % 32) .. + 3
#pragma unroll
  for (int j = 0; j < 16; ++j) vv[j] = rsrc_load4(vrs, ((32 * wave + 2 * j + hh) * D + 4 * (lane % 32)) * 4);
  __builtin_amdgcn_sched_barrier(0);
  // queries in base-2 logit units
  if (qlive) {
    float* qd = &qs[0][0] + 4 * threadIdx.x;
    qd[0] = q4.x * a.scale2;
    qd[1] = q4.y * a.scale2;
    qd[2] = q4.z * a.scale2;
    qd[3] = q4.w * a.scale2;
  }
  __syncthreads();  // queries in LDS
  float dot[2][kSufMaxHeads];
#pragma unroll
  for (uint32_t h = 0; h < kSufMaxHeads; ++h) {
    float acc0 = 0.f, acc1 = 0.f;
    if (h < gq) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float4 q = *reinterpret_cast<const float4*>(&qs[h][16 * i + 4 * kq]);
        acc0 = fmaf(q.x, kv[i].x, acc0);
        acc0 = fmaf(q.y, kv[i].y, acc0);
        acc0 = fmaf(q.z, kv[i].z, acc0);
        acc0 = fmaf(q.w, kv[i].w, acc0);
        acc1 = fmaf(q.x, kv[8 + i].x, acc1);
        acc1 = fmaf(q.y, kv[8 + i].y, acc1);
        acc1 = fmaf(q.z, kv[8 + i].z, acc1);
        acc1 = fmaf(q.w, kv[8 + i].w, acc1);
      }
    }
    dot[0][h] = quad_sum(acc0);
    dot[1][h] = quad_sum(acc1);
  }
  if (kq == 0) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const uint32_t r = 16 * p + qd4;  // row within the wave
#pragma unroll
      for (uint32_t h = 0; h < kSufMaxHeads; ++h)
        if (h < gq) sp[h][(r & 1) * 64 + 16 * wave + r / 2] = 32 * wave + r < n ? dot[p][h] : -INFINITY;
    }
  }
  __syncthreads();
  // softmax per head over the run's tokens (waves take heads w, w + 4)
  for (uint32_t h = wave; h < gq; h += 4) {
    const float s0 = sp[h][lane], s1 = sp[h][lane + 64];
    float m = fmaxf(s0, s1);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    const float p0 = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s0 - m);
    const float p1 = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s1 - m);
    float l = p0 + p1;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) l += __shfl_xor(l, o);
    sp[h][lane] = p0;
    sp[h][lane + 64] = p1;
    if (lane == 0) {
      ml[h][0] = m;
      ml[h][1] = l;
    }
  }
  __syncthreads();
  // value sums of this half-wave's 16 rows
  float4 acc[kSufMaxHeads];
#pragma unroll
  for (uint32_t h = 0; h < kSufMaxHeads; ++h) acc[h] = make_float4(0.f, 0.f, 0.f, 0.f);
  // a half-wave's 16 weights per head are contiguous (the order sp is written in): four rows'
  // weights per 16-byte read
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float4 p4[kSufMaxHeads];
#pragma unroll
    for (uint32_t h = 0; h < kSufMaxHeads; ++h)
      if (h < gq) p4[h] = reinterpret_cast<const float4*>(&sp[h][hh * 64 + 16 * wave])[i];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const float4 x = vv[4 * i + jj];
#pragma unroll
      for (uint32_t h = 0; h < kSufMaxHeads; ++h) {
        if (h < gq) {
          const float p = jj == 0 ? p4[h].x : jj == 1 ? p4[h].y : jj == 2 ? p4[h].z : p4[h].w;  // 0 past n
          acc[h].x = fmaf(p, x.x, acc[h].x);
          acc[h].y = fmaf(p, x.y, acc[h].y);
          acc[h].z = fmaf(p, x.z, acc[h].z);
          acc[h].w = fmaf(p, x.w, acc[h].w);
        }
      }
    }
  }
#pragma unroll
  for (uint32_t h = 0; h < kSufMaxHeads; ++h)
    if (h < gq) *reinterpret_cast<float4*>(&red[wave][hh][h][4 * (lane % 32)]) = acc[h];
  __syncthreads();
  for (uint32_t h = wave; h < gq; h += 4) {
    float2 o = make_float2(0.f, 0.f);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const float2 x = *reinterpret_cast<const float2*>(&red[w][half][h][2 * lane]);
        o.x += x.x;
        o.y += x.y;
      }
    }
    if constexpr (MERGED) {
      merge_suffix_row(a, sess, unit, h, lane, ml[h][0], ml[h][1], o);
    } else {
      float* part = a.ws + (uint64_t)sess * a.ws_sess_stride +
                    (((uint64_t)unit * a.nsplit_total + a.nsplit_fast + run) * gq + h) * (D + 2);
      *reinterpret_cast<float2*>(part + 2 * lane) = o;
      if (lane == 0) {
        part[D] = ml[h][0];
        part[D + 1] = ml[h][1];
      }
    }
  }
}

// Log-sum-exp merge of the split partials. One wave per output row (session, unit, head), or
// `parts` waves (2 or 4) that take every parts-th split and meet in LDS. Lane l owns channels
// l, l + 64, ... (CPL of them); the splits' (m, l) are wave-uniform loads, so each weight
// exp2(m - max) is computed once per wave, not once per channel. Loads go out in rounds of
// BATCH / CPL splits, all independent.
constexpr uint32_t kMergeThreads = 256;  // 4 waves
constexpr uint32_t kMergeBatchSmall = 32;  // loads per lane in flight per round: 16 splits at CPL 2
constexpr uint32_t kMergeBatchLarge = 48;  // 24 splits at CPL 2
constexpr uint32_t kMergeFewRows = 256;    // below this many rows the merge is latency-bound

// Rows of a decode token the attention launch consumed from its inputs, written to the key
// residual and the value window once that launch is over (null k: nothing to write).
struct PendRows {
  const float* k;
  const float* v;
  float* kres;
  float* vring;
  uint32_t kslot, vslot, R;
};

template <int CPL, uint32_t BATCH>
__global__ void __launch_bounds__(kMergeThreads)
    k_attn_merge(const float* ws, uint32_t nsplit, uint32_t parts, uint32_t gq, uint32_t D, uint32_t heads,
                 uint32_t qh, float* out, uint32_t units, uint32_t rows, uint64_t ws_sess_stride,
                 uint64_t out_sess_stride, PendRows pend) {
  constexpr uint32_t SB = BATCH / CPL;
  __shared__ float xch[4][2 + 64 * CPL];  // per wave: (m, l), then the channel sums
  const uint32_t lane = threadIdx.x % 64;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  const uint32_t row = blockIdx.x * (4 / parts) + wave / parts, part = wave % parts;
  const bool live = row < rows;
  float mp = -INFINITY, lp = 0.f, acc[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i) acc[i] = 0.f;
  uint32_t sess = 0, unit = 0, h = 0;
  // a decode token's rows (one wave per unit writes them at the end): requested first, so
  // their round trip overlaps the partials' loads
  float pk[CPL], pv[CPL];
  bool pend_rows = false;
  if (live) {
    sess = row / (units * gq);
    unit = (row / gq) % units;
    h = row % gq;
    pend_rows = pend.k != nullptr && sess == 0 && h == 0 && part == 0;
    if (pend_rows) {
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const uint32_t d = lane + 64 * i;
        pk[i] = d < D ? pend.k[(uint64_t)unit * D + d] : 0.f;
        pv[i] = d < D ? pend.v[(uint64_t)unit * D + d] : 0.f;
      }
    }
    const uint64_t stride = (uint64_t)gq * (D + 2);
    const float* base = ws + sess * ws_sess_stride + (uint64_t)unit * nsplit * stride + h * (D + 2);
    for (uint32_t s0 = part; s0 < nsplit; s0 += parts * SB) {
      float v[SB][CPL], ms[SB], ls[SB];
#pragma unroll
      for (uint32_t j = 0; j < SB; ++j) {
        const uint32_t s = s0 + j * parts;
        const float* ps = base + (uint64_t)(s < nsplit ? s : part) * stride;
        ms[j] = s < nsplit ? ps[D] : -INFINITY;
        ls[j] = ps[D + 1];
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
          const uint32_t c = lane + 64 * i;
          v[j][i] = ps[c < D ? c : 0];
        }
      }
      float bm = mp;
#pragma unroll
      for (uint32_t j = 0; j < SB; ++j) bm = fmaxf(bm, ms[j]);
      if (bm != -INFINITY) {
        const float r = __builtin_amdgcn_exp2f(mp - bm);  // 0 while mp is -inf
        lp *= r;
#pragma unroll
        for (int i = 0; i < CPL; ++i) acc[i] *= r;
#pragma unroll
        for (uint32_t j = 0; j < SB; ++j) {
          const float f = ms[j] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ms[j] - bm);
          lp = fmaf(ls[j], f, lp);
#pragma unroll
          for (int i = 0; i < CPL; ++i) acc[i] = fmaf(v[j][i], f, acc[i]);
        }
        mp = bm;
      }
    }
  }
  if (parts > 1) {
    if (lane == 0) {
      xch[wave][0] = mp;
      xch[wave][1] = lp;
    }
#pragma unroll
    for (int i = 0; i < CPL; ++i) xch[wave][2 + lane + 64 * i] = acc[i];
    __syncthreads();
    if (part == 0 && live) {
      float M = -INFINITY;
      for (uint32_t q = 0; q < parts; ++q) M = fmaxf(M, xch[wave + q][0]);
      lp = 0.f;
#pragma unroll
      for (int i = 0; i < CPL; ++i) acc[i] = 0.f;
      for (uint32_t q = 0; q < parts; ++q) {
        const float mq = xch[wave + q][0];
        const float f = mq == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mq - M);
        lp = fmaf(xch[wave + q][1], f, lp);
#pragma unroll
        for (int i = 0; i < CPL; ++i) acc[i] = fmaf(xch[wave + q][2 + lane + 64 * i], f, acc[i]);
      }
    }
  }
  if (part != 0 || !live) return;
  const uint32_t b = unit / heads, kvh = unit % heads;
  float* o = out + sess * out_sess_stride + ((uint64_t)b * qh + kvh * gq + h) * D;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const uint32_t c = lane + 64 * i;
    if (c < D) o[c] = acc[i] / lp;
  }
  if (pend_rows) {
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const uint32_t d = lane + 64 * i;
      if (d < D) {
        pend.kres[((uint64_t)unit * pend.R + pend.kslot) * D + d] = pk[i];
        pend.vring[((uint64_t)unit * pend.R + pend.vslot) * D + d] = pv[i];
      }
    }
  }
}

// Merge launch for `count` sessions of `units` units. Few rows (a latency-bound launch): four
// waves per row. Otherwise as few waves per row as one round of loads each allows (fewer
// waves and LDS exchanges for the same bytes).
hipError_t launch_merge(const float* ws, uint32_t nsplit, uint32_t gq, uint32_t D, uint32_t heads,
                        uint32_t qh, float* out, uint32_t units, uint32_t count,
                        uint64_t ws_sess_stride, uint64_t out_sess_stride, hipStream_t stream,
                        PendRows pend = PendRows{}) {
  const uint32_t cpl = D <= 64 ? 1 : D <= 128 ? 2 : D <= 256 ? 4 : D <= 512 ? 8 : 16;
  const uint32_t rows = count * units * gq;
  const uint32_t sb = (rows < kMergeFewRows ? kMergeBatchSmall : kMergeBatchLarge) / cpl;
  const uint32_t want = (nsplit + sb - 1) / sb;
  const uint32_t parts = want <= 1 ? 1 : want <= 2 ? 2 : 4;
  // the smaller round when it holds a wave's splits (fewer padded loads), else the larger
  const bool small = (nsplit + parts - 1) / parts <= kMergeBatchSmall / cpl;
  const uint32_t grid = (rows * parts + 3) / 4;
#define KIVI_MERGE(C)                                                                          \
  if (small)                                                                                   \
    k_attn_merge<C, kMergeBatchSmall><<<grid, kMergeThreads, 0, stream>>>(                     \
        ws, nsplit, parts, gq, D, heads, qh, out, units, rows, ws_sess_stride, out_sess_stride, pend); \
  else                                                                                         \
    k_attn_merge<C, kMergeBatchLarge><<<grid, kMergeThreads, 0, stream>>>(                     \
        ws, nsplit, parts, gq, D, heads, qh, out, units, rows, ws_sess_stride, out_sess_stride, pend)
  switch (cpl) {
    case 1: KIVI_MERGE(1); break;
    case 2: KIVI_MERGE(2); break;
    case 4: KIVI_MERGE(4); break;
    case 8: KIVI_MERGE(8); break;
    default: KIVI_MERGE(16); break;
  }
#undef KIVI_MERGE
  return hipGetLastError();
}

// ------------------------------------------------------------------ shared-prefix GEMM splits
// Batched sessions over one prefix: a unit's rows are all its (session, GQA head) pairs (64
// sessions x 4 heads = 256 rows), so each packed chunk is the shared operand of a real GEMM.
// A workgroup of 8 waves owns 256 rows (32 per wave). It dequantizes each 64-token chunk of
// keys and values into LDS once (f32 dequant at a power-of-two range, split into hi + lo f16),
// and every wave runs
//   S^T[64 t][32 r]   = K[t][d]   . Q^T[d][r]     (v_mfma_f32_32x32x16_f16)
//   O^T[128 d][32 r] += V^T[d][t] . P^T[t][r]
// with hi/lo operands on both sides (a*b ~ ah*bh + ah*bl + al*bh: ~22-bit products, f32
// sums). A row is the MFMA N index (lane % 32) in both products, so one lane pair (lanes r
// and r + 32) owns a row's logits, softmax state and outputs.
//
// Pipeline (one barrier per chunk): while the waves run the MFMAs of chunk c from LDS buffer
// c%2, they dequantize chunk c+1 into buffer (c+1)%2 from code words already in registers and
// (scale, zero) already in LDS, and the loads of chunk c+2 are in flight.

typedef _Float16 hx8 __attribute__((ext_vector_type(8)));
typedef float fx16 __attribute__((ext_vector_type(16)));

constexpr uint32_t kShThreads = 512;   // 8 waves
constexpr uint32_t kShRows = 256;      // rows per workgroup (32 per wave)
constexpr uint32_t kShKRow = 128 + 8;  // K LDS row (one token) stride in halves, padded
constexpr uint32_t kShVRow = 64 + 8;   // V^T LDS row (one channel) stride in halves, padded
constexpr uint32_t kShBufHalves = 2 * 64 * kShKRow + 2 * 128 * kShVRow;  // khi, klo, vhi, vlo
constexpr uint32_t kShParamFloats = 1024;  // keys [2 groups][128][2], values [4 groups][64][2]
constexpr size_t kShLdsBytes = 2 * (size_t)kShBufHalves * sizeof(_Float16) + 2 * kShParamFloats * sizeof(float);
// P operands are p * 2^kShPExp with p <= 2^kShSlack (below 2^14); the f16 subnormal floor of
// the lo halves then costs at most 2^-(kShPExp + 25) per token against a row sum l >= 1.
constexpr float kShSlack = 6.f;
constexpr float kShPExp = 8.f;
constexpr float kShPScale = 256.f;  // 2^kShPExp
static_assert(kShSlack + kShPExp <= 14.f, "P operands stay below 2^14");
constexpr uint32_t kShOutRow = 128 + 4;  // partial row (acc[128], m, l) in LDS, 16 B aligned
static_assert((size_t)kShRows * kShOutRow * sizeof(float) <= kShLdsBytes, "partials fit the chunk buffers");

typedef uint32_t ux4 __attribute__((ext_vector_type(4)));

// hi + lo f16 pairs of two floats (hi rounded toward zero, lo = f16(x - hi) rounded to
// nearest: ~22 significant bits). Returns (hi pair, lo pair).
__device__ __forceinline__ uint2 split2(float x, float y) {
  const uint32_t h = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(x, y));
  return make_uint2(h, lo_pair(x, y, h));
}

__device__ __forceinline__ fx16 mfma32(const hx8& a, const hx8& b, const fx16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Power-of-two factor 2^e with |x| * 2^e < 2^14 for |x| <= amax.
__device__ __forceinline__ int range_exp(float amax) {
  return std::min(60, std::max(-100, 14 - __builtin_amdgcn_frexp_expf(amax)));
}

// One chunk's global data as a thread holds it between its load and its dequant: the key
// words of tokens 2tp, 2tp+1 for channels 8o..8o+7; the value words of channel c, tokens
// 16j..16j+15; threads 0..255 also carry one float4 of the chunk's (scale, zero) block.
template <int BITS>
struct ShRaw {
  static constexpr int KW = BITS == 8 ? 2 : 1;  // words per token per channel octet
  static constexpr int VW = BITS / 2;           // words per channel per 16 tokens
  uint32_t k[2][KW];
  uint32_t v[VW];
  float4 prm;
};

// Per-thread base pointers of a unit's chunk data (chunk 0); chunk c adds c times the
// per-chunk strides, which are the same for every thread.
template <int BITS>
struct ShSrc {
  const uint32_t* k;  // key words of tokens 2tp, 2tp+1, channel octet o
  const uint32_t* v;  // value words of channel c, tokens 16j..
  const float4* p;    // one float4 of the chunk's (scale, zero) block
  static constexpr uint32_t kStride = 64 * (128 * BITS / 32);  // words per chunk, keys
  static constexpr uint32_t vStride = 128 * (64 * BITS / 32);  // words per chunk, values
  static constexpr uint32_t pStride = 128;                      // float4 per chunk, either kind
};

template <int BITS>
__device__ __forceinline__ ShSrc<BITS> shared_src(const AttnArgs& a, uint32_t unit) {
  constexpr uint32_t D = 128, PPW = 32 / BITS, KWT = D / PPW, VWC = 64 / PPW;
  const Geometry& g = a.c.geo;
  const uint32_t tid = threadIdx.x;
  const uint32_t o = tid % 16, tp = tid / 16, c = tid % 128, j = tid / 128;
  ShSrc<BITS> src;
  src.k = a.c.kcodes + unit * g.kcodes_unit() + (uint64_t)(2 * tp) * KWT + (BITS == 8 ? 2 * o : BITS == 4 ? o : o / 2);
  src.v = a.c.vcodes + unit * g.vcodes_unit() + c * VWC + j * (BITS / 2);
  // (scale, zero): keys [2 groups][128][2] and values [4 groups][64][2] are each 512
  // contiguous floats per chunk; threads 128..255 take values, the others keys (threads
  // 256.. load a key float4 again and drop it, so there is no branch around the load)
  src.p = (tid >= 128 && tid < 256)
              ? reinterpret_cast<const float4*>(a.c.vparams + unit * g.vparams_unit()) + (tid - 128)
              : reinterpret_cast<const float4*>(a.c.kparams + unit * g.kparams_unit()) + tid % 128;
  return src;
}

template <int BITS>
__device__ __forceinline__ void shared_load(const ShSrc<BITS>& src, uint32_t chunk, ShRaw<BITS>& raw) {
  constexpr uint32_t KWT = 128 * BITS / 32;
  const uint32_t* kw = src.k + (uint64_t)chunk * ShSrc<BITS>::kStride;
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    if constexpr (BITS == 8) {
      const uint2 w = *reinterpret_cast<const uint2*>(kw + x * KWT);
      raw.k[x][0] = w.x;
      raw.k[x][1] = w.y;
    } else {
      raw.k[x][0] = kw[x * KWT];
    }
  }
  const uint32_t* vw = src.v + (uint64_t)chunk * ShSrc<BITS>::vStride;
  if constexpr (BITS == 8) {
    const uint4 w = *reinterpret_cast<const uint4*>(vw);
    raw.v[0] = w.x; raw.v[1] = w.y; raw.v[2] = w.z; raw.v[3] = w.w;
  } else if constexpr (BITS == 4) {
    const uint2 w = *reinterpret_cast<const uint2*>(vw);
    raw.v[0] = w.x; raw.v[1] = w.y;
  } else {
    raw.v[0] = vw[0];
  }
  raw.prm = src.p[(uint64_t)chunk * ShSrc<BITS>::pStride];
}

// (scale, zero) into LDS, pre-multiplied by the range factor of keys (kf) or values (vf)
// (exact: powers of two), so the dequant is one fma per element.
template <int BITS>
__device__ __forceinline__ void shared_store_params(const ShRaw<BITS>& raw, float kf, float vf, float* prm) {
  if (threadIdx.x < 256) {
    const float f = threadIdx.x < 128 ? kf : vf;
    reinterpret_cast<float4*>(prm)[threadIdx.x] =
        make_float4(raw.prm.x * f, raw.prm.y * f, raw.prm.z * f, raw.prm.w * f);
  }
}

// Dequantize one chunk into a buffer: keys as [64 tokens][kShKRow] hi and lo, values as
// [128 channels][kShVRow] hi and lo with the tokens permuted so that a lane's 8 MFMA K-slots
// are 8 consecutive halves: position 16j + 8h + i holds token 16j + 8(i/4) + 4h + i%4 (bits 2
// and 3 swapped), the order in which the S^T output leaves the probabilities in a lane.
template <int BITS>
__device__ __forceinline__ void shared_dequant(const ShRaw<BITS>& raw, const float* prm, _Float16* buf) {
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  _Float16* khi = buf;
  _Float16* klo = khi + 64 * kShKRow;
  _Float16* vhi = klo + 64 * kShKRow;
  _Float16* vlo = vhi + 128 * kShVRow;
  const uint32_t tid = threadIdx.x;
  {
    const uint32_t o = tid % 16, tp = tid / 16;
    const float4* pk = reinterpret_cast<const float4*>(prm + ((tp / 16) * 128 + 8 * o) * 2);
    float sc[8], zr[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 v = pk[q];
      sc[2 * q] = v.x; zr[2 * q] = v.y;
      sc[2 * q + 1] = v.z; zr[2 * q + 1] = v.w;
    }
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      float d[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        uint32_t code;
        if constexpr (BITS == 8) code = (raw.k[x][e / 4] >> (8 * (e % 4))) & MASK;
        else if constexpr (BITS == 4) code = (raw.k[x][0] >> code_shift(4, e)) & MASK;
        else code = (raw.k[x][0] >> (2 * (o % 2) + 4 * e)) & MASK;  // elements 8(o%2) + e
        d[e] = fmaf(static_cast<float>(code), sc[e], zr[e]);
      }
      ux4 hi, lo;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
      const uint2 t2 = split2(d[2 * q], d[2 * q + 1]);
      hi[q] = t2.x;
      lo[q] = t2.y;
    }
      *reinterpret_cast<ux4*>(khi + (2 * tp + x) * kShKRow + 8 * o) = hi;
      *reinterpret_cast<ux4*>(klo + (2 * tp + x) * kShKRow + 8 * o) = lo;
    }
  }
  {
    const uint32_t c = tid % 128, j = tid / 128;
    const float4* pv = reinterpret_cast<const float4*>(prm + 512 + ((c / 32) * 64 + 16 * j) * 2);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float d[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int k = 8 * (i / 4) + 4 * h + i % 4;  // token within the 16-token run
        uint32_t code;
        if constexpr (BITS == 8) code = (raw.v[k / 4] >> (8 * (k % 4))) & MASK;
        else if constexpr (BITS == 4) code = (raw.v[k / 8] >> code_shift(4, k % 8)) & MASK;
        else code = (raw.v[0] >> code_shift(2, k)) & MASK;
        const float4 p = pv[k / 2];
        d[i] = fmaf(static_cast<float>(code), k % 2 ? p.z : p.x, k % 2 ? p.w : p.y);
      }
      ux4 hi, lo;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
      const uint2 t2 = split2(d[2 * q], d[2 * q + 1]);
      hi[q] = t2.x;
      lo[q] = t2.y;
    }
      *reinterpret_cast<ux4*>(vhi + c * kShVRow + 16 * j + 8 * h) = hi;
      *reinterpret_cast<ux4*>(vlo + c * kShVRow + 16 * j + 8 * h) = lo;
    }
  }
}

// Logits of one chunk for a wave's 32 rows: S^T tiles of tokens r and 32 + r.
__device__ __forceinline__ void shared_logits(const _Float16* buf, const hx8 (&qhi)[8], const hx8 (&qlo)[8],
                                              fx16& s0, fx16& s1) {
  const uint32_t lane = threadIdx.x % 64, h = lane / 32, r = lane % 32;
  const _Float16* khi = buf;
  const _Float16* klo = khi + 64 * kShKRow;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    s0[v] = 0.f;
    s1[v] = 0.f;
  }
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const hx8 kh0 = *reinterpret_cast<const hx8*>(khi + r * kShKRow + 16 * s + 8 * h);
    const hx8 kl0 = *reinterpret_cast<const hx8*>(klo + r * kShKRow + 16 * s + 8 * h);
    const hx8 kh1 = *reinterpret_cast<const hx8*>(khi + (32 + r) * kShKRow + 16 * s + 8 * h);
    const hx8 kl1 = *reinterpret_cast<const hx8*>(klo + (32 + r) * kShKRow + 16 * s + 8 * h);
    s0 = mfma32(kh0, qhi[s], s0);
    s1 = mfma32(kh1, qhi[s], s1);
    s0 = mfma32(kh0, qlo[s], s0);
    s1 = mfma32(kh1, qlo[s], s1);
    s0 = mfma32(kl0, qhi[s], s0);
    s1 = mfma32(kl1, qhi[s], s1);
  }
}

// Online softmax of one chunk's logits and the value mix for a wave's 32 rows.
__device__ __forceinline__ void shared_mix(const _Float16* buf, fx16 s0, fx16 s1,
                                           float s_unscale, float& m, float& l, fx16 (&o)[4],
                                           uint32_t valid = 64) {
  const uint32_t lane = threadIdx.x % 64, h = lane / 32, r = lane % 32;
  if (valid < 64) {
    // S^T value v of tile T is token 32T + 8(v/4) + 4h + v%4 of the chunk
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const uint32_t t = 8 * (v / 4) + 4 * h + v % 4;
      if (t >= valid) s0[v] = -INFINITY;
      if (32 + t >= valid) s1[v] = -INFINITY;
    }
  }
  const _Float16* vhi = buf + 2 * 64 * kShKRow;
  const _Float16* vlo = vhi + 128 * kShVRow;
  // online softmax over the chunk (the lane pair r, r + 32 holds the row's 64 logits) against
  // a reference maximum m that moves only when a row's chunk maximum exceeds it by more than
  // kShSlack: then every row of the wave takes max(m, chunk maximum) and rescales what it has
  // summed. The probabilities p = 2^(x - m) <= 2^kShSlack come out as p * kShPScale (the P
  // operand range), and so does l.
  float mx = -INFINITY;
#pragma unroll
  for (int v = 0; v < 16; ++v) mx = fmaxf(mx, fmaxf(s0[v], s1[v]));
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  const float cm = mx * s_unscale;
  if (__ballot(cm > m + kShSlack)) {  // wave-uniform
    const float mnew = fmaxf(m, cm);
    const float alpha = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mnew);
    m = mnew;
    l *= alpha;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int v = 0; v < 16; ++v) o[mt][v] *= alpha;
  }
  const float off = kShPExp - m;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    // P^T K-step j: tokens 16j .. 16j + 15 = tile j/2, values 8(j%2) .. 8(j%2) + 7
    float p[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float sv = j < 2 ? s0[8 * (j % 2) + i] : s1[8 * (j % 2) + i];
      p[i] = __builtin_amdgcn_exp2f(fmaf(sv, s_unscale, off));
      l += p[i];
    }
    ux4 ph, pl;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint2 t2 = split2(p[2 * q], p[2 * q + 1]);
      ph[q] = t2.x;
      pl[q] = t2.y;
    }
    const hx8 phh = __builtin_bit_cast(hx8, ph), pll = __builtin_bit_cast(hx8, pl);
    hx8 vh[4], vl[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      vh[mt] = *reinterpret_cast<const hx8*>(vhi + (32 * mt + r) * kShVRow + 16 * j + 8 * h);
      vl[mt] = *reinterpret_cast<const hx8*>(vlo + (32 * mt + r) * kShVRow + 16 * j + 8 * h);
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) o[mt] = mfma32(vh[mt], phh, o[mt]);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) o[mt] = mfma32(vh[mt], pll, o[mt]);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) o[mt] = mfma32(vl[mt], phh, o[mt]);
  }
}

// A prefix chunk that holds fp32 rows (the key residual / value window band), dequantized
// directly into buffer `buf` (no pipelining; these are the last one or two chunks of a
// prefix): tokens below kq / vq from the packed arrays, the rest from the residual / ring;
// tokens from `seq` on are zero (and masked in the softmax).
template <int BITS>
__device__ void shared_dequant_mixed(const AttnArgs& a, uint32_t unit, uint32_t chunk, float kf, float vf,
                                     _Float16* buf) {
  constexpr uint32_t D = 128, PPW = 32 / BITS, KWT = D / PPW, VWC = 64 / PPW, MASK = (1u << BITS) - 1u;
  const Geometry& g = a.c.geo;
  const uint64_t kq = a.st.kq, vq = a.st.vq, seq = a.seq;
  const uint32_t R = g.R;
  _Float16* khi = buf;
  _Float16* klo = khi + 64 * kShKRow;
  _Float16* vhi = klo + 64 * kShKRow;
  _Float16* vlo = vhi + 128 * kShVRow;
  const uint32_t tid = threadIdx.x;
  {
    const uint32_t o = tid % 16, tp = tid / 16;
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      const uint64_t t = (uint64_t)chunk * 64 + 2 * tp + x;
      float d[8];
      if (t < kq) {
        const float4* pk = reinterpret_cast<const float4*>(a.c.kparams + unit * g.kparams_unit() + (t / 32) * D * 2 + 16 * o);
        const uint32_t* wp = a.c.kcodes + unit * g.kcodes_unit() + t * KWT;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t ch = 8 * o + e;
          const uint32_t code = (wp[ch / PPW] >> code_shift(BITS, ch % PPW)) & MASK;
          const float4 p = pk[e / 2];
          d[e] = fmaf(static_cast<float>(code), e % 2 ? p.z : p.x, e % 2 ? p.w : p.y) * kf;
        }
      } else if (t < seq) {
        const float4* r = reinterpret_cast<const float4*>(a.c.kres + ((uint64_t)unit * R + (t - kq)) * D + 8 * o);
        const float4 r0 = r[0], r1 = r[1];
        d[0] = r0.x * kf; d[1] = r0.y * kf; d[2] = r0.z * kf; d[3] = r0.w * kf;
        d[4] = r1.x * kf; d[5] = r1.y * kf; d[6] = r1.z * kf; d[7] = r1.w * kf;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) d[e] = 0.f;
      }
      ux4 hi, lo;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint2 t2 = split2(d[2 * q], d[2 * q + 1]);
        hi[q] = t2.x;
        lo[q] = t2.y;
      }
      *reinterpret_cast<ux4*>(khi + (2 * tp + x) * kShKRow + 8 * o) = hi;
      *reinterpret_cast<ux4*>(klo + (2 * tp + x) * kShKRow + 8 * o) = lo;
    }
  }
  {
    const uint32_t c = tid % 128, j = tid / 128;
    const float2* vp = reinterpret_cast<const float2*>(a.c.vparams + unit * g.vparams_unit()) +
                       ((uint64_t)chunk * g.ncg() + c / 32) * 64;
    const uint32_t* wc = a.c.vcodes + unit * g.vcodes_unit() + (uint64_t)chunk * D * VWC + c * VWC;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float d[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t k = 16 * j + 8 * (i / 4) + 4 * h + i % 4;  // token within the chunk
        const uint64_t t = (uint64_t)chunk * 64 + k;
        if (t < vq) {
          const uint32_t code = (wc[k / PPW] >> code_shift(BITS, k % PPW)) & MASK;
          const float2 p = vp[k];
          d[i] = fmaf(static_cast<float>(code), p.x, p.y) * vf;
        } else if (t < seq) {
          d[i] = a.c.vring[((uint64_t)unit * R + (a.st.vhead + (t - vq)) % R) * D + c] * vf;
        } else {
          d[i] = 0.f;
        }
      }
      ux4 hi, lo;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint2 t2 = split2(d[2 * q], d[2 * q + 1]);
        hi[q] = t2.x;
        lo[q] = t2.y;
      }
      *reinterpret_cast<ux4*>(vhi + c * kShVRow + 16 * j + 8 * h) = hi;
      *reinterpret_cast<ux4*>(vlo + c * kShVRow + 16 * j + 8 * h) = lo;
    }
  }
}

// One workgroup: rows [rblk*256, +256) of `unit` over the packed chunks of split `split` (a
// contiguous range), partials into split index `split` of each row's session.
template <int BITS>
__device__ __forceinline__ void shared_split(const AttnArgs& a, uint32_t unit, uint32_t rblk,
                                             uint32_t split, uint8_t* lds) {
  constexpr uint32_t D = 128;
  _Float16* bufs = reinterpret_cast<_Float16*>(lds);  // [2][kShBufHalves]
  float* prms = reinterpret_cast<float*>(lds + 2 * (size_t)kShBufHalves * sizeof(_Float16));  // [2][1024]
  const uint32_t lane = threadIdx.x % 64, wave = threadIdx.x / 64, h = lane / 32, r = lane % 32;
  const uint32_t gq = a.gq;
  const uint32_t row = rblk * kShRows + wave * 32 + r;
  const uint32_t sess = row / gq, head = row % gq;
  const bool live = sess < a.nsess;
  const uint32_t b = unit / a.heads, kvh = unit % a.heads;

  // q of the lane's row, channels 16s + 8h + i, in base-2 logit units, split hi/lo at a
  // per-row power-of-two range
  const float* qp = a.query + (uint64_t)(live ? sess : 0) * a.q_sess_stride +
                    ((uint64_t)b * a.qh + kvh * gq + head) * D + 8 * h;
  const float qs = live ? a.scale2 : 0.f;
  float qf[8][8];
  float qmax = 0.f;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const float4 v0 = *reinterpret_cast<const float4*>(qp + 16 * s);
    const float4 v1 = *reinterpret_cast<const float4*>(qp + 16 * s + 4);
    qf[s][0] = v0.x * qs; qf[s][1] = v0.y * qs; qf[s][2] = v0.z * qs; qf[s][3] = v0.w * qs;
    qf[s][4] = v1.x * qs; qf[s][5] = v1.y * qs; qf[s][6] = v1.z * qs; qf[s][7] = v1.w * qs;
#pragma unroll
    for (int i = 0; i < 8; ++i) qmax = fmaxf(qmax, fabsf(qf[s][i]));
  }
  qmax = fmaxf(qmax, __shfl_xor(qmax, 32));
  const int eq = range_exp(qmax);
  const float qfac = ldexpf(1.f, eq);
  hx8 qhi[8], qlo[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    ux4 hi, lo;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint2 t2 = split2(qf[s][2 * q] * qfac, qf[s][2 * q + 1] * qfac);
      hi[q] = t2.x;
      lo[q] = t2.y;
    }
    qhi[s] = __builtin_bit_cast(hx8, hi);
    qlo[s] = __builtin_bit_cast(hx8, lo);
  }
  const int ek = range_exp(unit_max(a.c, unit, kMaxKeyAbs));
  const int ev = range_exp(unit_max(a.c, unit, kMaxValueAbs));
  const float kf = ldexpf(1.f, ek), vf = ldexpf(1.f, ev);
  const float s_unscale = ldexpf(1.f, -ek - eq);
  const float o_unscale = ldexpf(1.f, -ev) / kShPScale;  // O and l carry the P operand scale

  // contiguous chunk ranges over [0, gemm_end); chunks from chunk_end on hold fp32 rows
  const uint32_t cps = (a.gemm_end + a.nsplit_fast - 1) / a.nsplit_fast;
  const uint32_t c0 = std::min(a.gemm_end, split * cps);
  const uint32_t c1 = std::min(a.gemm_end, c0 + cps);
  const uint32_t p1 = std::min(c1, a.chunk_end);  // packed part [c0, p1)
  float m = -INFINITY, l = 0.f;
  fx16 o[4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[mt][v] = 0.f;

  if (c0 < p1) {
    // Chunks past the packed range's end are clamped to its last chunk: their loads stay in bounds and
    // their dequant goes to the buffer no later iteration reads.
    const ShSrc<BITS> src = shared_src<BITS>(a, unit);
    ShRaw<BITS> cur, nxt;
    shared_load<BITS>(src, c0, cur);
    shared_store_params<BITS>(cur, kf, vf, prms + (c0 % 2) * kShParamFloats);
    __syncthreads();
    shared_dequant<BITS>(cur, prms + (c0 % 2) * kShParamFloats, bufs + (c0 % 2) * kShBufHalves);
    shared_load<BITS>(src, std::min(c0 + 1, p1 - 1), cur);
    shared_store_params<BITS>(cur, kf, vf, prms + ((c0 + 1) % 2) * kShParamFloats);
    __syncthreads();
    // Top of iteration c: buffer c%2 holds chunk c; params (c+1)%2 and `cur` hold chunk c+1.
    // The dequant of chunk c+1 comes first, so `cur` is dead before the logit registers are
    // live (no spills at 256 VGPRs).
    for (uint32_t c = c0; c < p1; ++c) {
      shared_load<BITS>(src, std::min(c + 2, p1 - 1), nxt);
      const _Float16* buf = bufs + (c % 2) * kShBufHalves;
      shared_dequant<BITS>(cur, prms + ((c + 1) % 2) * kShParamFloats, bufs + ((c + 1) % 2) * kShBufHalves);
      fx16 s0, s1;
      shared_logits(buf, qhi, qlo, s0, s1);
      shared_mix(buf, s0, s1, s_unscale, m, l, o);
      shared_store_params<BITS>(nxt, kf, vf, prms + (c % 2) * kShParamFloats);
      cur = nxt;
      __syncthreads();
    }
  }
  // the prefix's fp32 band (the split covering the last chunks): direct dequant, masked tail
  for (uint32_t c = std::max(c0, a.chunk_end); c < c1; ++c) {
    shared_dequant_mixed<BITS>(a, unit, c, kf, vf, bufs);
    __syncthreads();
    fx16 s0, s1;
    shared_logits(bufs, qhi, qlo, s0, s1);
    const uint64_t left = a.seq - (uint64_t)c * 64;
    shared_mix(bufs, s0, s1, s_unscale, m, l, o, left < 64 ? static_cast<uint32_t>(left) : 64u);
    __syncthreads();  // the buffer is rewritten by the next chunk
  }
  l += __shfl_xor(l, 32);
  // Partials through LDS, so that the global stores are whole rows of consecutive lanes:
  // (acc[128], m, l) of the wave's row r at LDS row r of its block (stride kShOutRow floats).
  float* ob = reinterpret_cast<float*>(lds) + (size_t)wave * 32 * kShOutRow;
  __syncthreads();  // every wave is done with the chunk buffers
  // O^T value v of tile mt is channel 32mt + 8(v/4) + 4h + v%4
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4)
      *reinterpret_cast<float4*>(ob + r * kShOutRow + 32 * mt + 8 * q4 + 4 * h) =
          make_float4(o[mt][4 * q4] * o_unscale, o[mt][4 * q4 + 1] * o_unscale, o[mt][4 * q4 + 2] * o_unscale,
                      o[mt][4 * q4 + 3] * o_unscale);
  if (h == 0) {
    ob[r * kShOutRow + D] = c1 > c0 ? m : -INFINITY;
    ob[r * kShOutRow + D + 1] = c1 > c0 ? l / kShPScale : 0.f;
  }
  __syncthreads();
  // row rr of the wave, float2 f of its 65: the partial of (session, head) at its workspace row
  const uint32_t row0 = rblk * kShRows + wave * 32;
  for (uint32_t i = lane; i < 32 * 65; i += 64) {
    const uint32_t rr = i / 65, f = i % 65;
    const uint32_t rg = row0 + rr, se = rg / gq, hd = rg % gq;
    if (se < a.nsess) {
      float* part = a.ws + (uint64_t)se * a.ws_sess_stride + (((uint64_t)unit * a.nsplit_total + split) * gq + hd) * (D + 2);
      *reinterpret_cast<float2*>(part + 2 * f) = *reinterpret_cast<const float2*>(ob + rr * kShOutRow + 2 * f);
    }
  }
}

// Batched sessions, GEMM form: one workgroup per (unit, 256-row block, split) of the packed
// prefix chunks, for all sessions' rows at once. The split ranges are contiguous; the row
// blocks of one split are nsplit_fast apart in the grid (a multiple of the XCD count when
// nsplit_fast is), so they share an L2.
template <int BITS>
__global__ void __launch_bounds__(kShThreads) k_attn_shared(AttnArgs a) {
  extern __shared__ float lds[];
  const uint32_t rblocks = (a.nsess * a.gq + kShRows - 1) / kShRows;
  const uint32_t unit = blockIdx.x / (rblocks * a.nsplit_fast);
  const uint32_t rem = blockIdx.x % (rblocks * a.nsplit_fast);
  shared_split<BITS>(a, unit, rem / a.nsplit_fast, rem % a.nsplit_fast, reinterpret_cast<uint8_t*>(lds));
}

// ------------------------------------------------------------------ planning

uint32_t split_tokens(uint32_t gq) {
  uint32_t s = 256;
  while (s > 32 && (uint64_t)gq * s > 8192) s >>= 1;
  return s;
}

// Shapes of the matrix-core path: head_dim 64, 128, 192 or 256, G = 32 or a multiple of 64 (a
// chunk's half-waves then read one key group), any GQA, above one row set in head groups (of 8,
// or 4 above head_dim 128) that each read the chunks.
bool fast_eligible(const AttnProblem& p) {
  const Geometry& g = p.cache.geo;
  const uint32_t gq = p.qh / p.heads;
  const bool dim_ok = g.D == 64 || g.D == 128 || g.D == 192 || g.D == 256;
  return dim_ok && (g.G == 32 || g.G % 64 == 0) && (g.bits == 2 || g.bits == 4 || g.bits == 8) && gq >= 1;
}
// MFMA row sets (4 heads each) per workgroup, and the head groups of a unit
int fast_nrs(uint32_t D, uint32_t gq) { return D > 128 || gq <= 4 ? 1 : 2; }
// Eight-head groups at head_dim 128 and G = 32 take the 16x16x32 kernel for their packed chunks.
bool wide_shape(const AttnProblem& p) {
  const uint32_t gq = p.qh / p.heads;
  return fast_eligible(p) && p.cache.geo.D == 128 && p.cache.geo.G == 32 && fast_nrs(128, gq) == 2;
}
// GQA a multiple of 16 at head_dim 128 and G = 32: packed splits on the sixteen-head kernel.
bool wide16_shape(const AttnProblem& p) {
  const uint32_t gq = p.qh / p.heads;
  return fast_eligible(p) && p.cache.geo.D == 128 && p.cache.geo.G == 32 && gq % 16 == 0;
}
uint32_t head_groups(uint32_t D, uint32_t gq) {
  const uint32_t per = 4u * static_cast<uint32_t>(fast_nrs(D, gq));
  return (gq + per - 1) / per;
}

// MFMA chunks: [0, floor(vq/64)) (keys and values packed; vq <= kq). Everything after
// (value window, its band of packed keys, session suffix) goes to the generic kernel.
AttnArgs make_args(const AttnProblem& p, float* ws) {
  AttnArgs a{};
  a.c = p.cache;
  a.st = p.st;
  a.pend_k = p.pend_k;
  a.pend_v = p.pend_v;
  a.pend_vslot = p.pend_vslot;
  a.pend_evict = p.pend_k != nullptr ? p.pend_evict : 0u;
  a.seq = p.seq;
  a.L = p.suffix_len;
  a.total = p.seq + p.suffix_len;
  a.suffix_k = p.suffix_k;
  a.suffix_v = p.suffix_v;
  a.suffix_stride = p.suffix_stride;
  a.query = p.query;
  a.qh = p.qh;
  a.heads = p.heads;
  a.gq = p.qh / p.heads;
  a.scale2 = p.scale * kLog2e;
  // The MFMA path covers every 64-token chunk once some keys are packed: chunks
  // [0, floor(vq/64)) (keys and values all packed) in one launch, the rest (the fp32 value
  // window and key residual, the session suffix) in a second launch of the MIXED kernel.
  // Without packed keys, or for other shapes, the generic splits cover everything.
  // At head_dim 64 and 256 the MFMA launch takes only the fully packed chunks and the generic
  // splits the rest.
  const bool fast = fast_eligible(p) && p.st.kq > 0;
  const bool fast_win = fast && p.cache.geo.D == 128;
  a.S = split_tokens(a.gq);
  a.chunk_begin = 0;
  a.chunk_end = fast ? static_cast<uint32_t>(std::min(p.st.kq, p.st.vq) / 64) : 0;
  a.win_begin = a.chunk_end;
  a.win_end = fast_win ? static_cast<uint32_t>((a.total + 63) / 64) : a.chunk_end;
  a.hgroups = fast ? head_groups(p.cache.geo.D, a.gq) : 1u;
  a.gshift = fast ? static_cast<uint32_t>(__builtin_ctz(p.cache.geo.G)) : 5u;
  a.wide = !(fast && wide_shape(p)) ? 0u : wide16_shape(p) ? 2u : 1u;
  a.hgroups_fast = a.wide == 2 ? a.gq / kWide16Heads : a.hgroups;
  // packed splits per unit: at most kFastCpw (wide_cpw) chunks per wave, at least one, and at
  // least kFastGroups workgroups (over units and head groups) when the chunks allow
  {
    const uint32_t units = p.cache.geo.units * a.hgroups_fast;
    const uint32_t cpw = a.wide == 2 ? static_cast<uint32_t>(kWide16Cpw)
                         : a.wide ? static_cast<uint32_t>(wide_cpw(static_cast<int>(p.cache.geo.bits)))
                                  : static_cast<uint32_t>(fast_cpw(static_cast<int>(p.cache.geo.bits), fast_nrs(p.cache.geo.D, a.gq)));
    const uint32_t fewest = (a.chunk_end + 4 * cpw - 1) / (4 * cpw);
    const uint32_t most = (a.chunk_end + 3) / 4;
    a.nsplit_fast = std::min(most, std::max(fewest, (kFastGroups + units - 1) / units));
  }
  a.nsplit_win = a.win_end - a.win_begin;  // one chunk per workgroup, a quarter per wave
  a.t_begin = fast_win ? a.total : fast ? (uint64_t)a.chunk_end * 64 : 0;
  if (fast && !fast_win) {
    // the rest is short (the fp32 residual and window, a suffix): shorter splits, down to 16
    // tokens while the rest would fill fewer than ~1024 workgroups
    a.S = std::max(32u, a.S / 4);
    const uint64_t rest = a.total - a.t_begin;
    while (a.S > 16 && (uint64_t)p.cache.geo.units * ((rest + a.S - 1) / a.S) < 1024) a.S >>= 1;
  }
  a.nsplit_gen = static_cast<uint32_t>((a.total - a.t_begin + a.S - 1) / a.S);
  a.nsplit_total = a.nsplit_fast + a.nsplit_win + a.nsplit_gen;
  a.ws = ws;
  a.out = p.out;
  a.units = p.cache.geo.units;
  a.nsess = 0;
  a.gemm_end = 0;
  a.q_sess_stride = a.ws_sess_stride = 0;
  return a;
}

// A launch whose waves own at most one packed chunk each (at head_dim 128, where the window
// chunks are MIXED workgroups of one chunk anyway) takes the SMALL instantiation.
bool small_launch(const AttnArgs& a) {
  return a.c.geo.D == 128 && a.gq <= 4 && (uint64_t)a.nsplit_fast * 4 >= a.chunk_end - a.chunk_begin;
}

template <int BITS, int NRS, int D>
hipError_t launch_fast(const AttnArgs& a, double bytes, hipStream_t stream) {
  constexpr int NH = 4 * NRS;
  const bool small = D == 128 && NRS == 1 && small_launch(a);
  const size_t logits = (size_t)4 * NH * ((a.nsplit_fast > 0 && !small ? fast_cpw(BITS, NRS) : 1) * 64 + kRowPad);
  const size_t combine = (size_t)4 * NH * (D + 2);
  const size_t gen = a.nsplit_gen > 0 ? (size_t)a.gq * (D + a.S) : 0;  // generic splits' q and weights
  const size_t lds = std::max(std::max(logits, combine), gen) * sizeof(float);
  TimedLaunch timed(KIVI_KERNEL_ATTN_PACKED, stream, bytes);
  const uint32_t grid = a.units * (a.hgroups * a.nsplit_win + a.hgroups_fast * a.nsplit_fast + a.nsplit_gen);
  if constexpr (D == 128 && NRS == 2) {
    if (a.wide == 2) {
      const size_t wide = (size_t)4 * kWide16Heads * (kWide16Cpw * 64 + kRowPad);
      const size_t mixed = (size_t)4 * NH * (64 + kRowPad);
      const size_t comb16 = (size_t)4 * kWide16Heads * (D + 2);
      const size_t wlds = std::max(std::max(wide, mixed), comb16) * sizeof(float);
      k_attn_wide16<BITS><<<grid, kThreads, wlds, stream>>>(a);
      return hipGetLastError();
    }
    if (a.wide) {
      const size_t wide = (size_t)4 * kWideHeads * (wide_cpw(BITS) * 64 + kRowPad);
      const size_t mixed = (size_t)4 * NH * (64 + kRowPad);
      const size_t wlds = std::max(std::max(wide, mixed), combine) * sizeof(float);
      if (a.pend_evict)
        k_attn_wide<BITS, true><<<grid, kThreads, wlds, stream>>>(a);
      else
        k_attn_wide<BITS, false><<<grid, kThreads, wlds, stream>>>(a);
      return hipGetLastError();
    }
  }
  if constexpr (D == 128 && NRS == 1) {
    if (small) {
      k_attn_mfma<BITS, NRS, D, true><<<grid, kThreads, lds, stream>>>(a);
      return hipGetLastError();
    }
  }
  k_attn_mfma<BITS, NRS, D><<<grid, kThreads, lds, stream>>>(a);
  return hipGetLastError();
}

hipError_t dispatch_fast(const AttnArgs& a, double bytes, hipStream_t stream) {
  const uint32_t D = a.c.geo.D;
  const int nrs = fast_nrs(D, a.gq);
  switch (D * 100 + a.c.geo.bits * 10 + nrs) {
    case 12821: return launch_fast<2, 1, 128>(a, bytes, stream);
    case 12822: return launch_fast<2, 2, 128>(a, bytes, stream);
    case 12841: return launch_fast<4, 1, 128>(a, bytes, stream);
    case 12842: return launch_fast<4, 2, 128>(a, bytes, stream);
    case 12881: return launch_fast<8, 1, 128>(a, bytes, stream);
    case 12882: return launch_fast<8, 2, 128>(a, bytes, stream);
    case 6421: return launch_fast<2, 1, 64>(a, bytes, stream);
    case 6422: return launch_fast<2, 2, 64>(a, bytes, stream);
    case 6441: return launch_fast<4, 1, 64>(a, bytes, stream);
    case 6442: return launch_fast<4, 2, 64>(a, bytes, stream);
    case 6481: return launch_fast<8, 1, 64>(a, bytes, stream);
    case 6482: return launch_fast<8, 2, 64>(a, bytes, stream);
    case 19221: return launch_fast<2, 1, 192>(a, bytes, stream);
    case 19241: return launch_fast<4, 1, 192>(a, bytes, stream);
    case 19281: return launch_fast<8, 1, 192>(a, bytes, stream);
    case 25621: return launch_fast<2, 1, 256>(a, bytes, stream);
    case 25641: return launch_fast<4, 1, 256>(a, bytes, stream);
    case 25681: return launch_fast<8, 1, 256>(a, bytes, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t dispatch_generic(const AttnArgs& a, hipStream_t stream) {
  const size_t lds = ((size_t)a.gq * a.c.geo.D + (size_t)a.gq * a.S) * sizeof(float);
  k_attn_generic<0, 0, 0><<<a.units * a.nsplit_gen, kThreads, lds, stream>>>(a);
  return hipGetLastError();
}

}  // namespace

// The static workspace. In host code `scratch` is only a stand-in for the symbol: its device
// address on each device comes from hipGetSymbolAddress, never from the name.
static __device__ __align__(256) float scratch[kStaticWorkspaceFloats];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch[kMaxDevices] = {};

__global__ void __launch_bounds__(kThreads) k_fill_zero(float* out, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    out[i] = 0.f;
}

}  // namespace

hipError_t static_workspace(float** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (p == nullptr) return hipErrorInvalidSymbol;
    g_scratch[dev] = static_cast<float*>(p);
  }
  *out = g_scratch[dev];
  return hipSuccess;
}

hipError_t launch_fill_zero(float* out, size_t n, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  const size_t blocks = std::min<size_t>((n + kThreads - 1) / kThreads, 1024);
  k_fill_zero<<<static_cast<unsigned>(blocks), kThreads, 0, stream>>>(out, n);
  return hipGetLastError();
}

// The decode fused into the attention launch quantizes the evicted window token with the
// 32-channel value groups of one half-wave, once per chunk workgroup: G = 32, one head group
// (up to four heads on the 4x4x4 kernel, five to eight on the 16x16x32 one).
bool attention_fuses_decode(const AttnProblem& p) {
  const AttnArgs a = make_args(p, nullptr);
  return a.total > 0 && a.nsplit_gen == 0 && (a.nsplit_fast > 0 || a.nsplit_win > 0) &&
         p.cache.geo.D == 128 && p.cache.geo.G == 32 && a.hgroups == 1;
}

size_t attention_workspace_floats(const AttnProblem& p) {
  const AttnArgs a = make_args(p, nullptr);
  return (size_t)p.cache.geo.units * a.nsplit_total * a.gq * (p.cache.geo.D + 2);
}

hipError_t launch_attention(const AttnProblem& p, float* workspace, hipStream_t stream) {
  AttnArgs a = make_args(p, workspace);
  if (a.total == 0) return hipSuccess;
  const Geometry& g = p.cache.geo;
  const uint32_t units = g.units;
  // algorithmic bytes per token of one unit: packed codes + (scale, zero), or fp32 rows
  const double key_tok = g.D * g.bits / 8.0 + g.D * 8.0 / g.G;
  const double val_tok = g.D * g.bits / 8.0 + g.ncg() * 8.0;
  const double row = g.D * 4.0;
  const double q_bytes = (double)units * a.gq * g.D * 4.0;
  const uint64_t t0 = a.t_begin, kq = p.st.kq, vq = p.st.vq;
  const double kp = kq > t0 ? (double)(kq - t0) : 0.0, vp = vq > t0 ? (double)(vq - t0) : 0.0;
  const double kd = (double)(p.seq - std::max(kq, t0)), vd = (double)(p.seq - std::max(vq, t0));
  const double tail_bytes = units * (kp * key_tok + vp * val_tok + (kd + vd + 2.0 * p.suffix_len) * row);
  if (a.nsplit_fast > 0 || a.nsplit_win > 0) {
    // one launch over every chunk (the tokens after the packed chunks as window chunks at
    // head_dim 128, as generic splits in the same grid otherwise): packed tokens at packed
    // cost, the rest as fp32 rows
    const double kpt = (double)std::min<uint64_t>(kq, p.seq), vpt = (double)vq;
    const double fp32_rows = (double)(p.seq - kq) + (double)(p.seq - vq) + 2.0 * p.suffix_len;
    hipError_t e = dispatch_fast(
        a, units * (kpt * key_tok + vpt * val_tok + fp32_rows * row) + q_bytes, stream);
    if (e != hipSuccess) return e;
  } else {
    TimedLaunch timed(KIVI_KERNEL_ATTN_TAIL, stream, tail_bytes + q_bytes);
    hipError_t e = dispatch_generic(a, stream);
    if (e != hipSuccess) return e;
  }
  const double bytes = (double)units * a.gq * ((double)a.nsplit_total * (g.D + 2) + g.D) * 4.0;
  TimedLaunch timed(KIVI_KERNEL_ATTN_MERGE, stream, bytes);
  PendRows pend{};
  if (p.pend_k != nullptr)
    pend = PendRows{p.pend_k, p.pend_v, p.cache.kres, p.cache.vring, p.pend_kslot, p.pend_vslot, g.R};
  return launch_merge(workspace, a.nsplit_total, a.gq, g.D, p.heads, p.qh, p.out, units, 1, 0, 0,
                      stream, pend);
}

namespace {

// Arguments of one launch group as one problem over the prefix (the window range is sized
// for the group's longest suffix; each session clips it to its own).
AttnArgs make_session_args(const SessionsProblem& sp, uint32_t nsess, uint64_t max_suffix, float* ws) {
  AttnProblem p{};
  p.cache = sp.cache;
  p.st = sp.st;
  p.seq = sp.seq;
  p.suffix_len = max_suffix;
  p.query = sp.queries;
  p.out = sp.out;
  p.qh = sp.qh;
  p.heads = sp.heads;
  p.batch = sp.batch;
  p.scale = sp.scale;
  AttnArgs a = make_args(p, ws);
  a.nsplit_fast = (a.chunk_end + 4 * kSessCpw - 1) / (4 * kSessCpw);
  a.nsplit_total = a.nsplit_fast + a.nsplit_win + a.nsplit_gen;
  a.nsess = nsess;
  a.q_sess_stride = (uint64_t)sp.batch * sp.qh * sp.cache.geo.D;
  a.ws_sess_stride = (uint64_t)sp.cache.geo.units * a.nsplit_total * a.gq * (sp.cache.geo.D + 2);
  return a;
}

bool sessions_supported(const SessionsProblem& sp) {
  AttnProblem p{};
  p.cache = sp.cache;
  p.st = sp.st;
  p.qh = sp.qh;
  p.heads = sp.heads;
  // the batched-sessions kernels take head_dim 128, G = 32 and GQA <= 8
  return sp.n > 0 && fast_eligible(p) && sp.st.kq > 0 && sp.cache.geo.D == 128 && sp.cache.geo.G == 32 &&
         sp.qh / sp.heads <= 8;
}

uint64_t longest_suffix(const SessionsProblem& sp, uint32_t first, uint32_t count) {
  uint64_t m = 0;
  for (uint32_t i = first; i < first + count; ++i) m = std::max<uint64_t>(m, sp.sessions[i].len);
  return m;
}

// Rows (sessions x GQA heads) from which one launch group takes the GEMM form: below it a
// 32-row MFMA tile would be mostly padding and the per-session form does less work.
constexpr uint32_t kSharedMinRows = 16;
// Workgroups the GEMM form aims for (one per CU: 148 KB of LDS each).
constexpr uint32_t kSharedTargetGroups = 256;

bool use_shared(const SessionsProblem& sp, uint32_t nsess) {
  return nsess * (sp.qh / sp.heads) >= kSharedMinRows;
}

// The GEMM form's splits: the packed chunks of a unit in nsplit contiguous ranges, nsplit a
// multiple of 8 (the XCD count) where the chunks allow, so about kSharedTargetGroups
// workgroups cover units x row blocks x splits.
// The GEMM form covers every prefix chunk, [0, ceil(seq/64)) (the fp32 band of the prefix
// too, as the prefix's smax covers those rows); k_attn_suffix covers each session's suffix
// [seq, seq + len) in runs of kSufTokens.
AttnArgs make_shared_args(const SessionsProblem& sp, uint32_t nsess, uint64_t max_suffix, float* ws) {
  AttnArgs a = make_session_args(sp, nsess, max_suffix, ws);
  const uint32_t rblocks = (nsess * a.gq + kShRows - 1) / kShRows;
  const uint32_t per = a.units * rblocks;
  uint32_t ns = (kSharedTargetGroups + per - 1) / per;
  ns = (ns + 7) / 8 * 8;
  a.gemm_end = static_cast<uint32_t>((sp.seq + 63) / 64);
  a.nsplit_fast = a.gemm_end == 0 ? 0 : std::max(1u, std::min(ns, a.gemm_end));
  // suffixes: runs of kSufTokens tokens (k_attn_suffix)
  a.nsplit_win = static_cast<uint32_t>((max_suffix + kSufTokens - 1) / kSufTokens);
  a.nsplit_total = a.nsplit_fast + a.nsplit_win + a.nsplit_gen;
  a.ws_sess_stride = (uint64_t)sp.cache.geo.units * a.nsplit_total * a.gq * (sp.cache.geo.D + 2);
  return a;
}

// Algorithmic bytes of one launch group: the prefix's packed and fp32 rows, the sessions'
// suffix rows, and the queries.
struct GroupBytes {
  double prefix, suffixes, queries;
};

template <int BITS, int NRS>
hipError_t launch_sessions(const AttnArgs& a, const SessionTable& t, const GroupBytes& by,
                           hipStream_t stream) {
  constexpr int NH = 4 * NRS;
  const size_t logits = (size_t)4 * NH * ((a.nsplit_fast > 0 ? kSessCpw : 1) * 64 + kRowPad);
  const size_t combine = (size_t)4 * NH * (128 + 2);
  const size_t lds = std::max(logits, combine) * sizeof(float);
  const uint32_t grid = a.nsess * a.units * a.nsplit_win + a.units * a.nsplit_fast;
  TimedLaunch timed(KIVI_KERNEL_ATTN_SESSIONS, stream, by.prefix + by.suffixes + by.queries);
  k_attn_sessions<BITS, NRS><<<grid, kThreads, lds, stream>>>(a, t);
  return hipGetLastError();
}

// A launch group of the GEMM form whose suffixes fit one run (at most kSufTokens tokens each):
// its suffix kernel runs after k_attn_shared and merges every output row itself.
bool shared_merges_in_suffix(const AttnArgs& a) { return a.nsplit_fast > 0 && a.nsplit_win <= 1; }

template <int BITS, int NRS>
hipError_t launch_shared(const AttnArgs& a, const SessionTable& t, const GroupBytes& by,
                         hipStream_t stream) {
  const bool merged = shared_merges_in_suffix(a);
  // window / suffix chunks per session: one workgroup per (session, unit, run of suffix tokens)
  const uint32_t nwin = a.nsess * a.units * a.nsplit_win;
  if (nwin > 0 && !merged) {
    TimedLaunch timed(KIVI_KERNEL_ATTN_SESSIONS, stream, by.suffixes + by.queries);
    k_attn_suffix<false><<<nwin, kThreads, 0, stream>>>(a, t);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (a.nsplit_fast == 0) return hipSuccess;
  {
    const hipError_t e = raise_lds_limit(reinterpret_cast<const void*>(&k_attn_shared<BITS>), kShLdsBytes);
    if (e != hipSuccess) return e;
  }
  const uint32_t rblocks = (a.nsess * a.gq + kShRows - 1) / kShRows;
  {
    TimedLaunch timed(KIVI_KERNEL_ATTN_SHARED, stream, by.prefix + by.queries);
    k_attn_shared<BITS><<<a.units * rblocks * a.nsplit_fast, kShThreads, kShLdsBytes, stream>>>(a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || !merged) return e;
  }
  // the suffixes and the merge of every row: the suffix rows and queries, the GEMM partials
  // read back, the outputs written
  const double rows = (double)a.nsess * a.units * a.gq;
  TimedLaunch timed(KIVI_KERNEL_ATTN_SESSIONS, stream,
                    by.suffixes + by.queries + rows * ((double)a.nsplit_fast * (a.c.geo.D + 2) + a.c.geo.D) * 4.0);
  k_attn_suffix<true><<<a.nsess * a.units, kThreads, 0, stream>>>(a, t);
  return hipGetLastError();
}

}  // namespace

namespace {

// Launch group [first, first + count): its form and arguments (queries, outputs and the
// window range of that group).
AttnArgs group_args(const SessionsProblem& p, uint32_t first, uint32_t count, float* ws, bool* shared) {
  SessionsProblem gp = p;
  gp.queries = p.queries + (uint64_t)first * p.batch * p.qh * p.cache.geo.D;
  gp.out = p.out + (uint64_t)first * p.batch * p.qh * p.cache.geo.D;
  *shared = use_shared(p, count);
  const uint64_t longest = longest_suffix(p, first, count);
  return *shared ? make_shared_args(gp, count, longest, ws) : make_session_args(gp, count, longest, ws);
}

}  // namespace

size_t sessions_workspace_floats(const SessionsProblem& p) {
  if (!sessions_supported(p)) return 0;
  // every launch group reuses the workspace from its start
  size_t most = 0;
  for (uint32_t first = 0; first < p.n; first += kMaxLaunchSessions) {
    const uint32_t count = std::min(kMaxLaunchSessions, p.n - first);
    bool shared;
    const AttnArgs a = group_args(p, first, count, nullptr, &shared);
    most = std::max(most, (size_t)count * a.ws_sess_stride);
  }
  return most;
}

hipError_t launch_sessions_attention(const SessionsProblem& p, float* workspace,
                                     hipStream_t stream) {
  if (!sessions_supported(p)) return hipErrorNotSupported;
  const Geometry& g = p.cache.geo;
  for (uint32_t first = 0; first < p.n; first += kMaxLaunchSessions) {
    const uint32_t count = std::min(kMaxLaunchSessions, p.n - first);
    SessionTable t{};
    double suffix_rows = 0.0;
    for (uint32_t i = 0; i < count; ++i) {
      t.d[i] = p.sessions[first + i];
      suffix_rows += 2.0 * (double)t.d[i].len;
    }
    bool shared;
    const AttnArgs a = group_args(p, first, count, workspace, &shared);
    // algorithmic bytes: the prefix once, every session's suffix, the queries
    const double key_tok = g.D * g.bits / 8.0 + g.D * 8.0 / g.G;
    const double val_tok = g.D * g.bits / 8.0 + g.ncg() * 8.0;
    const double row = g.D * 4.0;
    const double fp32_rows = (double)(p.seq - p.st.kq) + (double)(p.seq - p.st.vq);
    const GroupBytes by{g.units * ((double)p.st.kq * key_tok + (double)p.st.vq * val_tok + fp32_rows * row),
                        g.units * suffix_rows * row, count * (double)a.q_sess_stride * 4.0};
    hipError_t e = hipSuccess;
    const int nrs = a.gq <= 4 ? 1 : 2;
    switch (g.bits * 10 + nrs) {
      case 21: e = shared ? launch_shared<2, 1>(a, t, by, stream) : launch_sessions<2, 1>(a, t, by, stream); break;
      case 22: e = shared ? launch_shared<2, 2>(a, t, by, stream) : launch_sessions<2, 2>(a, t, by, stream); break;
      case 41: e = shared ? launch_shared<4, 1>(a, t, by, stream) : launch_sessions<4, 1>(a, t, by, stream); break;
      case 42: e = shared ? launch_shared<4, 2>(a, t, by, stream) : launch_sessions<4, 2>(a, t, by, stream); break;
      case 81: e = shared ? launch_shared<8, 1>(a, t, by, stream) : launch_sessions<8, 1>(a, t, by, stream); break;
      case 82: e = shared ? launch_shared<8, 2>(a, t, by, stream) : launch_sessions<8, 2>(a, t, by, stream); break;
      default: e = hipErrorInvalidValue; break;
    }
    if (e != hipSuccess) return e;
    if (shared && shared_merges_in_suffix(a)) continue;  // the suffix kernel wrote the outputs
    const double bytes = (double)count * g.units * a.gq * ((double)a.nsplit_total * (g.D + 2) + g.D) * 4.0;
    TimedLaunch timed(KIVI_KERNEL_ATTN_MERGE, stream, bytes);
    e = launch_merge(workspace, a.nsplit_total, a.gq, g.D, p.heads, p.qh, a.out, g.units, count,
                     a.ws_sess_stride, a.q_sess_stride, stream);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace kivi
