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
// Two split kinds write one workspace of partials (m, l, acc[D]) per (unit, split, head):
//  * k_attn_mfma — every 64-token chunk whose keys AND values are packed
//    (tokens [0, 64*floor(vq/64))), for G=32, D=128, bits 2/4/8 and GQA <= 8. Both
//    contractions run on the matrix cores (v_mfma_f32_4x4x1_16B, fp32 products):
//      logits[h][t] = bias_g[h] + sum_d (q[h][d]*scale_g[d]) * code[d][t]
//      out[h][d]   += sum_t (w[h][t]*scale_t[cg]) * code[t][d] + sum_t w[h][t]*zero_t[cg]
//    The GQA heads are the 4 MFMA rows; the 16 4x4 blocks tile 64 tokens (keys) or 64
//    channels (values); CBSZ/ABID broadcast lets one A register feed 8 K-steps. A lane
//    owns a token (keys) or a channel (values), and the native layout packs exactly that
//    lane's codes into its words, so a word unpacks into 4-16 MFMA B operands.
//  * k_attn_generic — the remaining tokens (the fp32 window and its band of packed keys,
//    the session suffix) and every shape the MFMA kernel does not cover: one
//    thread per token in the reference's operation order (recon = fma(code, scale, zero);
//    logit = fma(recon, q, logit), channels ascending, src/attention.rs:143-177, 289-300).
#include "common.hpp"
#include "kivi.h"

#include <algorithm>

namespace kivi {
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
  // MFMA splits: chunks [chunk_begin, chunk_end) in workgroups of 4 waves x CPW chunks,
  // written to workspace splits split_base .. split_base + nsplit_launch - 1
  uint32_t chunk_begin;
  uint32_t chunk_end;
  uint32_t nsplit_launch;
  uint32_t split_base;
  uint32_t nsplit_fast;    // MFMA splits of both launches (generic splits follow them)
  uint32_t nsplit_total;   // splits per unit in the workspace
  float* ws;               // [units][nsplit_total][gq][D+2]
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
  const float code = static_cast<float>((word >> (bits * (d % ppw))) & ((1u << bits) - 1u));
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
  const float code = static_cast<float>((word >> (bits * (tt % ppw))) & ((1u << bits) - 1u));
  const float m = t < vq ? 1.f : 0.f;
  return fmaf(fmaf(code, sz.x, sz.y), m, dense * (1.f - m));  // exact for m in {0, 1}
}

__device__ __forceinline__ float warp_max(float v) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
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
__global__ void __launch_bounds__(kThreads) k_attn_generic(AttnArgs a) {
  extern __shared__ float lds[];
  const Geometry& g = a.c.geo;
  const uint32_t D = DD ? DD : g.D, gq = a.gq, S = a.S;
  const uint32_t unit = blockIdx.x / a.nsplit_gen;
  const uint32_t split = blockIdx.x % a.nsplit_gen;
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
  float* part = a.ws + ((uint64_t)unit * a.nsplit_total + a.nsplit_fast + split) * gq * (D + 2);
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

// ------------------------------------------------------------------ MFMA splits

constexpr int kRowPad = 4;  // floats of padding per logit row (LDS bank spread)

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

// Codes of one packed word as MFMA B operands: out[p] = code at bits [b*p, b*p+b) times
// `unit`. 2- and 4-bit codes are masked one per byte; a byte p < 16 read as fp8 e4m3 is
// exactly p*unit (subnormals and the first binade are linear), so v_cvt_pk_f32_fp8 turns
// two codes into two f32 per instruction. 8-bit codes use v_cvt_f32_ubyte0..3 (unit 1).
typedef float v2f __attribute__((ext_vector_type(2)));
template <int BITS>
__device__ __forceinline__ void unpack_word(uint32_t w, float* out) {
  if constexpr (BITS == 2) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int m = static_cast<int>((w >> (2 * k)) & 0x03030303u);  // positions k, k+4, k+8, k+12
      const v2f lo = __builtin_amdgcn_cvt_pk_f32_fp8(m, false);
      const v2f hi = __builtin_amdgcn_cvt_pk_f32_fp8(m, true);
      out[k] = lo.x;
      out[k + 4] = lo.y;
      out[k + 8] = hi.x;
      out[k + 12] = hi.y;
    }
  } else if constexpr (BITS == 4) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int m = static_cast<int>((w >> (4 * k)) & 0x0F0F0F0Fu);  // positions k, k+2, k+4, k+6
      const v2f lo = __builtin_amdgcn_cvt_pk_f32_fp8(m, false);
      const v2f hi = __builtin_amdgcn_cvt_pk_f32_fp8(m, true);
      out[k] = lo.x;
      out[k + 2] = lo.y;
      out[k + 4] = hi.x;
      out[k + 6] = hi.y;
    }
  } else {
    out[0] = static_cast<float>(w & 0xFFu);
    out[1] = static_cast<float>((w >> 8) & 0xFFu);
    out[2] = static_cast<float>((w >> 16) & 0xFFu);
    out[3] = static_cast<float>(w >> 24);
  }
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

// Everything one chunk's logits read from HBM: the lane token's code words and the
// (scale, zero) pairs of its group half for channels 16*la .. +15.
template <int BITS>
struct KeyData {
  uint32_t kw[128 * BITS / 32];
  float4 sz[8];
};

// Everything one chunk's value mix reads from HBM: the lane channel's code words for both
// channel halves, and (scale, zero) of tokens 8*la .. +7 for channel groups lc, lc+2.
template <int BITS>
struct ValueData {
  uint32_t vw[2][64 * BITS / 32];
  float4 sz[2][4];
};

template <int BITS>
__device__ __forceinline__ void load_key_data(const AttnArgs& a, uint32_t unit, uint32_t ch,
                                              uint32_t lane, uint32_t la, uint32_t lc,
                                              KeyData<BITS>& kd) {
  constexpr int KW = 128 * BITS / 32;
  const Geometry& g = a.c.geo;
  const float4* pp = reinterpret_cast<const float4*>(
      a.c.kparams + unit * g.kparams_unit() + ((uint64_t)(2 * ch + lc) * 128 + 16 * la) * 2);
#pragma unroll
  for (int j = 0; j < 8; ++j) kd.sz[j] = pp[j];
  load_words<KW>(a.c.kcodes + unit * g.kcodes_unit() + ((uint64_t)ch * 64 + lane) * KW, kd.kw);
}

template <int BITS>
__device__ __forceinline__ void load_value_data(const AttnArgs& a, uint32_t unit, uint32_t tb,
                                                uint32_t lane, uint32_t la, uint32_t lc,
                                                ValueData<BITS>& vd) {
  constexpr int VW = 64 * BITS / 32;
  const Geometry& g = a.c.geo;
#pragma unroll
  for (int hv = 0; hv < 2; ++hv) {
    load_words<VW>(a.c.vcodes + unit * g.vcodes_unit() + ((uint64_t)tb * 128 + lane + 64 * hv) * VW, vd.vw[hv]);
    const float4* pp = reinterpret_cast<const float4*>(
        a.c.vparams + unit * g.vparams_unit() + (((uint64_t)tb * 4 + lc + 2 * hv) * 64 + 8 * la) * 2);
#pragma unroll
    for (int j = 0; j < 4; ++j) vd.sz[hv][j] = pp[j];
  }
}

// Logits of one packed 64-token chunk for the lane's token (lane = token within the chunk).
// On gfx950 the 4x4 f32 MFMAs do not overlap VALU work, so each 16-channel step unpacks its
// codes (VALU block) and then issues its 16 MFMAs back to back (sched_barrier).
template <int BITS, int NRS>
__device__ __forceinline__ void chunk_logits(const KeyData<BITS>& kd, const float (&qv)[NRS][16],
                                             float unit_scale, float (&lg)[NRS][4]) {
  constexpr int PPW = 32 / BITS;
  float qp[NRS][16];
  float bias[NRS];
#pragma unroll
  for (int rs = 0; rs < NRS; ++rs) bias[rs] = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float4 sz = kd.sz[j];  // (s, z) of channels 2j, 2j+1
#pragma unroll
    for (int rs = 0; rs < NRS; ++rs) {
      qp[rs][2 * j] = qv[rs][2 * j] * sz.x;
      qp[rs][2 * j + 1] = qv[rs][2 * j + 1] * sz.z;
      bias[rs] = fmaf(qv[rs][2 * j], sz.y, bias[rs]);
      bias[rs] = fmaf(qv[rs][2 * j + 1], sz.w, bias[rs]);
    }
  }
#pragma unroll
  for (int rs = 0; rs < NRS; ++rs) bias[rs] = sum_over_blocks(bias[rs]) * unit_scale;
  v4f acc[NRS][2];
#pragma unroll
  for (int rs = 0; rs < NRS; ++rs) {
    acc[rs][0] = v4f{0.f, 0.f, 0.f, 0.f};
    acc[rs][1] = v4f{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int a2 = 0; a2 < 8; ++a2) {
    float code[16];
#pragma unroll
    for (int q = 0; q < 16 / PPW; ++q) unpack_word<BITS>(kd.kw[a2 * (16 / PPW) + q], code + q * PPW);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < 16; ++r)
#pragma unroll
      for (int rs = 0; rs < NRS; ++rs) acc[rs][r & 1] = mfma_bcast(qp[rs][r], code[r], acc[rs][r & 1], a2);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int rs = 0; rs < NRS; ++rs) {
    acc[rs][0] = mfma_bcast(bias[rs], 1.0f, acc[rs][0], 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) lg[rs][i] = acc[rs][0][i] + acc[rs][1][i];
  }
}

// Value mix of one packed 64-token chunk into vacc (lane = channel lane and 64+lane); w holds
// the lane's weights of tokens 8*la .. 8*la+7.
template <int BITS, int NRS>
__device__ __forceinline__ void chunk_values(const ValueData<BITS>& vd, const float (&w)[NRS][8],
                                             float inv_unit, v4f (&vacc)[NRS][2],
                                             float (&zacc)[NRS][2]) {
  constexpr int VW = 64 * BITS / 32, PPW = 32 / BITS;
  // A operands: w * scale / unit (the zero term is accumulated apart)
  float av[NRS][2][8];
#pragma unroll
  for (int hv = 0; hv < 2; ++hv) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float4 sz = vd.sz[hv][j];  // tokens 8*la + 2j, +1
#pragma unroll
      for (int rs = 0; rs < NRS; ++rs) {
        av[rs][hv][2 * j] = w[rs][2 * j] * inv_unit * sz.x;
        av[rs][hv][2 * j + 1] = w[rs][2 * j + 1] * inv_unit * sz.z;
        zacc[rs][hv] = fmaf(w[rs][2 * j], sz.y, zacc[rs][hv]);
        zacc[rs][hv] = fmaf(w[rs][2 * j + 1], sz.w, zacc[rs][hv]);
      }
    }
  }
  // both channel halves interleaved: two independent accumulation chains
#pragma unroll
  for (int q = 0; q < VW; ++q) {
    float code[2][PPW];
    unpack_word<BITS>(vd.vw[0][q], code[0]);
    unpack_word<BITS>(vd.vw[1][q], code[1]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int p = 0; p < PPW; ++p) {
      const int tt = q * PPW + p;  // token within the chunk: 8*a2 + r
      const int a2 = tt / 8, r = tt % 8;
#pragma unroll
      for (int hv = 0; hv < 2; ++hv)
#pragma unroll
        for (int rs = 0; rs < NRS; ++rs) vacc[rs][hv] = mfma_bcast(av[rs][hv][r], code[hv][p], vacc[rs][hv], a2);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// One workgroup = 4 waves; wave w of split s owns packed chunks [s*4*CPW + w*CPW, +CPW) of its
// unit (chunks whose 64 keys and 64 values are all packed). D = 128, G = 32.
template <int BITS, int NRS, int CPW>
__global__ void __launch_bounds__(kThreads) k_attn_mfma(AttnArgs a) {
  constexpr int D = 128;
  constexpr int ROW = CPW * 64 + kRowPad;  // logits row stride (floats)
  constexpr int NH = 4 * NRS;              // padded heads per unit
  extern __shared__ float lds[];
  const uint32_t unit = blockIdx.x / a.nsplit_launch;
  const uint32_t split = blockIdx.x % a.nsplit_launch;
  const uint32_t b = unit / a.heads, kvh = unit % a.heads;
  const uint32_t lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  const uint32_t la = (lane % 32) / 4;  // block within a half-wave
  const uint32_t li = lane % 4;         // MFMA row = head within the row set
  const uint32_t lc = lane / 32;        // half-wave: key group / value channel group parity
  const uint32_t gq = a.gq;
  float* wl = lds + wave * NH * ROW;    // this wave's logits [NH][ROW]

  // A byte p < 16 converted as fp8 is p * unit (unit = 2^-9 for OCP e4m3).
  const float unit_scale = BITS == 8 ? 1.f : __builtin_amdgcn_cvt_f32_fp8(1, 0);
  const float inv_unit = 1.f / unit_scale;  // exact power of two

  const int32_t c_begin = static_cast<int32_t>(a.chunk_begin + (split * 4 + wave) * CPW);
  const int32_t nch = std::max<int32_t>(0, std::min<int32_t>(CPW, static_cast<int32_t>(a.chunk_end) - c_begin));

  // q (base-2 logits, divided by the code unit) for the lane's head, channels 16*la .. +15.
  float qv[NRS][16];
#pragma unroll
  for (int rs = 0; rs < NRS; ++rs) {
    const uint32_t h = rs * 4 + li;
    const float* qp = a.query + ((uint64_t)b * a.qh + kvh * gq + min(h, gq - 1)) * D + 16 * la;
    const float s = h < gq ? a.scale2 * inv_unit : 0.f;
#pragma unroll
    for (int r = 0; r < 16; r += 4) {
      const float4 v = *reinterpret_cast<const float4*>(qp + r);
      qv[rs][r] = v.x * s;
      qv[rs][r + 1] = v.y * s;
      qv[rs][r + 2] = v.z * s;
      qv[rs][r + 3] = v.w * s;
    }
  }

  // ---------------- phase 1: logits of every owned chunk into LDS
  float mx[NRS][4];
#pragma unroll
  for (int rs = 0; rs < NRS; ++rs)
#pragma unroll
    for (int i = 0; i < 4; ++i) mx[rs][i] = -INFINITY;
  auto logits_of = [&](int k, const KeyData<BITS>& kd) {
    float lg[NRS][4];
    chunk_logits<BITS, NRS>(kd, qv, unit_scale, lg);
#pragma unroll
    for (int rs = 0; rs < NRS; ++rs)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        wl[(rs * 4 + i) * ROW + k * 64 + lane] = lg[rs][i];
        mx[rs][i] = fmaxf(mx[rs][i], lg[rs][i]);
      }
  };
  {
    // two register buffers: chunk k+1 is in flight while chunk k is computed
    KeyData<BITS> k0, k1;
    if (nch > 0) load_key_data<BITS>(a, unit, c_begin, lane, la, lc, k0);
    for (int k = 0; k < nch; k += 2) {
      if (k + 1 < nch) load_key_data<BITS>(a, unit, c_begin + k + 1, lane, la, lc, k1);
      logits_of(k, k0);
      if (k + 1 < nch) {
        if (k + 2 < nch) load_key_data<BITS>(a, unit, c_begin + k + 2, lane, la, lc, k0);
        logits_of(k + 1, k1);
      }
    }
  }
  // wave max per head; each lane keeps the max of its own MFMA row
  float mrow[NRS];
  float mall[NRS][4];
#pragma unroll
  for (int rs = 0; rs < NRS; ++rs) {
#pragma unroll
    for (int i = 0; i < 4; ++i) mall[rs][i] = warp_max(mx[rs][i]);
    mrow[rs] = li == 0 ? mall[rs][0] : li == 1 ? mall[rs][1] : li == 2 ? mall[rs][2] : mall[rs][3];
  }

  // ---------------- phase 2: value mix
  v4f vacc[NRS][2];
  float zacc[NRS][2];
  float lsum[NRS];
#pragma unroll
  for (int rs = 0; rs < NRS; ++rs) {
    vacc[rs][0] = v4f{0.f, 0.f, 0.f, 0.f};
    vacc[rs][1] = v4f{0.f, 0.f, 0.f, 0.f};
    zacc[rs][0] = zacc[rs][1] = 0.f;
    lsum[rs] = 0.f;
  }
  auto values_of = [&](int k, const ValueData<BITS>& vd) {
    float w[NRS][8];
#pragma unroll
    for (int rs = 0; rs < NRS; ++rs) {
      const float4* lp = reinterpret_cast<const float4*>(wl + (rs * 4 + li) * ROW + k * 64 + 8 * la);
      const float4 x0 = lp[0], x1 = lp[1];
      const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        w[rs][r] = __builtin_amdgcn_exp2f(xs[r] - mrow[rs]);  // v_exp_f32; argument <= 0
        lsum[rs] += w[rs][r];
      }
    }
    chunk_values<BITS, NRS>(vd, w, inv_unit, vacc, zacc);
  };
  {
    ValueData<BITS> v0, v1;
    if (nch > 0) load_value_data<BITS>(a, unit, c_begin, lane, la, lc, v0);
    for (int k = 0; k < nch; k += 2) {
      if (k + 1 < nch) load_value_data<BITS>(a, unit, c_begin + k + 1, lane, la, lc, v1);
      values_of(k, v0);
      if (k + 1 < nch) {
        if (k + 2 < nch) load_value_data<BITS>(a, unit, c_begin + k + 2, lane, la, lc, v0);
        values_of(k + 1, v1);
      }
    }
  }

  // ---------------- wave partial: reduce l and the zero terms over the 8 blocks
#pragma unroll
  for (int rs = 0; rs < NRS; ++rs) {
    lsum[rs] = sum_over_blocks(lsum[rs]);
    zacc[rs][0] = sum_over_blocks(zacc[rs][0]);
    zacc[rs][1] = sum_over_blocks(zacc[rs][1]);
  }
  __syncthreads();  // every wave is done with its logits; reuse LDS for the combine
  float* cw = lds + wave * NH * (D + 2);
#pragma unroll
  for (int rs = 0; rs < NRS; ++rs) {
#pragma unroll
    for (int hv = 0; hv < 2; ++hv) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // zero term of head i, channel group lc + 2*hv lives in lane 32*lc + i
        const float z = __shfl(zacc[rs][hv], 32 * lc + i);
        cw[(rs * 4 + i) * (D + 2) + lane + 64 * hv] = vacc[rs][hv][i] + z;
      }
    }
    if (lane < 4) {  // lanes 0..3 hold row li = lane after the reductions
      cw[(rs * 4 + lane) * (D + 2) + D] = nch > 0 ? mrow[rs] : -INFINITY;
      cw[(rs * 4 + lane) * (D + 2) + D + 1] = nch > 0 ? lsum[rs] : 0.f;
    }
  }
  __syncthreads();
  float* part = a.ws + ((uint64_t)unit * a.nsplit_total + a.split_base + split) * gq * (D + 2);
  for (uint32_t idx = threadIdx.x; idx < gq * (D + 2); idx += blockDim.x) {
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

// Log-sum-exp merge of the split partials: one workgroup per (unit, head). LDS holds the
// per-split factors 2^(m_s - M).
__global__ void __launch_bounds__(kThreads)
    k_attn_merge(const float* ws, uint32_t nsplit, uint32_t gq, uint32_t D, uint32_t heads,
                 uint32_t qh, float* out) {
  extern __shared__ float f_lds[];  // [nsplit] factors, then 8 reduction slots
  float* red = f_lds + nsplit;
  const uint32_t unit = blockIdx.x / gq, h = blockIdx.x % gq;
  const uint32_t b = unit / heads, kvh = unit % heads;
  const float* base = ws + (uint64_t)unit * nsplit * gq * (D + 2) + h * (D + 2);
  const uint64_t stride = (uint64_t)gq * (D + 2);
  const uint32_t lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  float m = -INFINITY;
  for (uint32_t s = threadIdx.x; s < nsplit; s += blockDim.x) m = fmaxf(m, base[s * stride + D]);
  m = warp_max(m);
  if (lane == 0) red[wave] = m;
  __syncthreads();
  const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float l = 0.f;
  for (uint32_t s = threadIdx.x; s < nsplit; s += blockDim.x) {
    const float ms = base[s * stride + D];
    const float f = ms == -INFINITY ? 0.f : exp2f(ms - M);
    f_lds[s] = f;
    l += base[s * stride + D + 1] * f;
  }
  l = warp_sum(l);
  if (lane == 0) red[4 + wave] = l;
  __syncthreads();
  const float inv = 1.0f / (red[4] + red[5] + red[6] + red[7]);
  float* o = out + ((uint64_t)b * qh + kvh * gq + h) * D;
  for (uint32_t d = threadIdx.x; d < D; d += blockDim.x) {
    float acc = 0.f;
    for (uint32_t s = 0; s < nsplit; ++s) acc = fmaf(base[s * stride + d], f_lds[s], acc);
    o[d] = acc * inv;
  }
}

// ------------------------------------------------------------------ planning

constexpr int kFastCpw = 8;  // chunks (64 tokens) per wave in the MFMA kernel

uint32_t split_tokens(uint32_t gq) {
  uint32_t s = 256;
  while (s > 32 && (uint64_t)gq * s > 8192) s >>= 1;
  return s;
}

bool fast_eligible(const AttnProblem& p) {
  const Geometry& g = p.cache.geo;
  const uint32_t gq = p.qh / p.heads;
  return g.D == 128 && g.G == 32 && (g.bits == 2 || g.bits == 4 || g.bits == 8) && gq >= 1 &&
         gq <= 8;
}

// MFMA chunks: [0, floor(vq/64)) (keys and values packed; vq <= kq). Everything after
// (value window, its band of packed keys, session suffix) goes to the generic kernel.
AttnArgs make_args(const AttnProblem& p, float* ws) {
  AttnArgs a{};
  a.c = p.cache;
  a.st = p.st;
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
  // the tail after the MFMA chunks is short: small splits give it enough workgroups
  a.S = fast_eligible(p) ? 16 : split_tokens(a.gq);
  a.chunk_begin = 0;
  a.chunk_end = fast_eligible(p) ? static_cast<uint32_t>(p.st.vq / 64) : 0;
  a.nsplit_fast = (a.chunk_end + 4 * kFastCpw - 1) / (4 * kFastCpw);
  a.nsplit_launch = a.nsplit_fast;
  a.split_base = 0;
  a.t_begin = (uint64_t)a.chunk_end * 64;
  a.nsplit_gen = static_cast<uint32_t>((a.total - a.t_begin + a.S - 1) / a.S);
  a.nsplit_total = a.nsplit_fast + a.nsplit_gen;
  a.ws = ws;
  return a;
}

template <int BITS, int NRS>
hipError_t launch_fast(const AttnArgs& a, hipStream_t stream) {
  constexpr int NH = 4 * NRS;
  const size_t logits = (size_t)4 * NH * (kFastCpw * 64 + kRowPad);
  const size_t combine = (size_t)4 * NH * (128 + 2);
  const size_t lds = std::max(logits, combine) * sizeof(float);
  k_attn_mfma<BITS, NRS, kFastCpw><<<a.c.geo.units * a.nsplit_fast, kThreads, lds, stream>>>(a);
  return hipGetLastError();
}

hipError_t dispatch_fast(const AttnArgs& a, hipStream_t stream) {
  const int nrs = a.gq <= 4 ? 1 : 2;
  switch (a.c.geo.bits * 10 + nrs) {
    case 21: return launch_fast<2, 1>(a, stream);
    case 22: return launch_fast<2, 2>(a, stream);
    case 41: return launch_fast<4, 1>(a, stream);
    case 42: return launch_fast<4, 2>(a, stream);
    case 81: return launch_fast<8, 1>(a, stream);
    case 82: return launch_fast<8, 2>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t dispatch_generic(const AttnArgs& a, bool fast_shape, hipStream_t stream) {
  const size_t lds = ((size_t)a.gq * a.c.geo.D + (size_t)a.gq * a.S) * sizeof(float);
  const dim3 grid(a.c.geo.units * a.nsplit_gen);
  if (!fast_shape) {
    k_attn_generic<0, 0, 0><<<grid, kThreads, lds, stream>>>(a);
  } else if (a.c.geo.bits == 2) {
    k_attn_generic<2, 128, 32><<<grid, kThreads, lds, stream>>>(a);
  } else if (a.c.geo.bits == 4) {
    k_attn_generic<4, 128, 32><<<grid, kThreads, lds, stream>>>(a);
  } else {
    k_attn_generic<8, 128, 32><<<grid, kThreads, lds, stream>>>(a);
  }
  return hipGetLastError();
}

}  // namespace

size_t attention_workspace_floats(const AttnProblem& p) {
  const AttnArgs a = make_args(p, nullptr);
  return (size_t)p.cache.geo.units * a.nsplit_total * a.gq * (p.cache.geo.D + 2);
}

hipError_t launch_attention(const AttnProblem& p, float* workspace, hipStream_t stream) {
  const AttnArgs a = make_args(p, workspace);
  if (a.total == 0) return hipSuccess;
  const Geometry& g = p.cache.geo;
  const uint32_t units = g.units;
  // algorithmic bytes per token of one unit: packed codes + (scale, zero), or fp32 rows
  const double key_tok = g.D * g.bits / 8.0 + g.D * 8.0 / g.G;
  const double val_tok = g.D * g.bits / 8.0 + g.ncg() * 8.0;
  const double row = g.D * 4.0;
  const double q_bytes = (double)units * a.gq * g.D * 4.0;
  if (a.nsplit_fast > 0) {
    const double tokens = (double)(a.chunk_end - a.chunk_begin) * 64;
    TimedLaunch timed(KIVI_KERNEL_ATTN_PACKED, stream, units * tokens * (key_tok + val_tok) + q_bytes);
    hipError_t e = dispatch_fast(a, stream);
    if (e != hipSuccess) return e;
  }
  if (a.nsplit_gen > 0) {
    const uint64_t t0 = a.t_begin, kq = p.st.kq, vq = p.st.vq;
    const double kp = kq > t0 ? (double)(kq - t0) : 0.0, vp = vq > t0 ? (double)(vq - t0) : 0.0;
    const double kd = (double)(p.seq - std::max(kq, t0)), vd = (double)(p.seq - std::max(vq, t0));
    const double bytes =
        units * (kp * key_tok + vp * val_tok + (kd + vd + 2.0 * p.suffix_len) * row) + q_bytes;
    TimedLaunch timed(KIVI_KERNEL_ATTN_TAIL, stream, bytes);
    hipError_t e = dispatch_generic(a, fast_eligible(p), stream);
    if (e != hipSuccess) return e;
  }
  const size_t merge_lds = ((size_t)a.nsplit_total + 8) * sizeof(float);
  {
    const double bytes = (double)units * a.gq * ((double)a.nsplit_total * (g.D + 2) + g.D) * 4.0;
    TimedLaunch timed(KIVI_KERNEL_ATTN_MERGE, stream, bytes);
    k_attn_merge<<<units * a.gq, kThreads, merge_lds, stream>>>(workspace, a.nsplit_total, a.gq,
                                                                g.D, p.heads, p.qh, p.out);
  }
  return hipGetLastError();
}

size_t sessions_workspace_floats(const SessionsProblem& p) {
  (void)p;
  return 0;
}

hipError_t launch_sessions_attention(const SessionsProblem& p, float* workspace,
                                     hipStream_t stream) {
  (void)p;
  (void)workspace;
  (void)stream;
  return hipErrorNotSupported;
}

}  // namespace kivi
