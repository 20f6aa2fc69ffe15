// kernels_quant.hip — KIVI quantization, residual/ring copies, stream export and
// dequantization on CDNA4 (gfx950).
//
// Bit-exactness with the reference (src/quant.rs:453-485): scale = span/levels and
// code = clamp(rint((x - zero)/scale), 0, levels) use IEEE-correct f32 division (hipcc's
// default; -ffast-math and reciprocal-multiply are never used) and v_rndne (round half to
// even, equal to the reference's floor-based rounding for every finite input). The value of
// a min/max does not depend on the reduction order; the sign of a zero minimum does, and
// follows the first-zero rule of common.hpp in every kernel here.
#include "common.hpp"
#include "kivi.h"

#include <algorithm>
#include <map>
#include <mutex>
#include <utility>

namespace kivi {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float scale_of(float span, float levels) {
  return span == 0.0f ? 0.0f : span / levels;
}

__device__ __forceinline__ uint32_t quant_code(float x, float zero, float scale, float levels) {
  if (scale == 0.0f) return 0u;
  float r = rintf((x - zero) / scale);
  if (r < 0.0f) {
    r = 0.0f;
  } else if (r > levels) {
    r = levels;
  }
  return static_cast<uint32_t>(r);
}

// Reciprocal for quant_code_fast: 0 for a zero scale (every code is then 0).
__device__ __forceinline__ float quant_inv(float scale) {
  return scale == 0.0f ? 0.0f : __builtin_amdgcn_rcpf(scale);
}

// quant_code from a reciprocal, bit-identical to it. With v_rcp_f32's 1-ulp reciprocal,
// q = (x - zero) * inv lies within q * 2^-22 <= 2^-14 of the correctly rounded quotient
// (x - zero) / scale (0 <= x - zero <= span keeps q <= levels (1 + 2^-22) <= 256), so both
// round to the same integer unless q is within 2^-12 of a half-integer: |q - rint(q)| >=
// 0.5 - 2^-12, which is also true of a non-finite q (inv = inf); those lanes divide.
// x >= zero here (zero is the group minimum), so r >= 0 and the clamp is an integer min.
__device__ __forceinline__ uint32_t quant_code_fast(float x, float zero, float scale, float inv,
                                                    uint32_t levels) {
#pragma clang fp contract(off)
  const float d = x - zero;
  const float q = d * inv;
  float r = rintf(q);
  if (!(fabsf(q - r) < 0.5f - 0x1p-12f)) r = scale == 0.0f ? 0.0f : rintf(d / scale);
  const uint32_t u = static_cast<uint32_t>(r);
  return u < levels ? u : levels;
}

// DPP lane exchanges inside rows of 16 lanes (every lane active): quad_perm xor 1 and xor 2,
// then mirrors that pair each lane with the other half of its 8- or 16-lane group.
constexpr int kDppXor1 = 0xB1;
constexpr int kDppXor2 = 0x4E;
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, true));
}

// min and max over aligned groups of L lanes (L a power of two, 1 <= L <= 64; wave-uniform),
// as compare-and-select (src/quant.rs:356 f32::min / max on finite values).
__device__ __forceinline__ void minmax_with(float& mn, float& mx, float omn, float omx) {
  mn = omn < mn ? omn : mn;
  mx = omx > mx ? omx : mx;
}
template <uint32_t L>
__device__ __forceinline__ void group_minmax(float& mn, float& mx) {
  if constexpr (L >= 2) minmax_with(mn, mx, dpp_f<kDppXor1>(mn), dpp_f<kDppXor1>(mx));
  if constexpr (L >= 4) minmax_with(mn, mx, dpp_f<kDppXor2>(mn), dpp_f<kDppXor2>(mx));
  if constexpr (L >= 8) minmax_with(mn, mx, dpp_f<kDppHalfMirror>(mn), dpp_f<kDppHalfMirror>(mx));
  if constexpr (L >= 16) minmax_with(mn, mx, dpp_f<kDppMirror>(mn), dpp_f<kDppMirror>(mx));
  if constexpr (L >= 32) minmax_with(mn, mx, __shfl_xor(mn, 16), __shfl_xor(mx, 16));
  if constexpr (L >= 64) minmax_with(mn, mx, __shfl_xor(mn, 32), __shfl_xor(mx, 32));
}

// v as held by lane p of the lane's 16-lane row (DPP row_newbcast).
__device__ __forceinline__ float row_bcast(float v, int p) {
  const int x = __float_as_int(v);
  switch (p) {
#define KIVI_RB(P) \
  case P: return __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x150 + P, 0xF, 0xF, true));
    KIVI_RB(0) KIVI_RB(1) KIVI_RB(2) KIVI_RB(3) KIVI_RB(4) KIVI_RB(5) KIVI_RB(6) KIVI_RB(7)
    KIVI_RB(8) KIVI_RB(9) KIVI_RB(10) KIVI_RB(11) KIVI_RB(12) KIVI_RB(13) KIVI_RB(14)
#undef KIVI_RB
    default: return __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x15F, 0xF, 0xF, true));
  }
}

// One exchange step of row_minmax16: of its n token pairs (lo[j], hi[j]) a lane keeps the lo
// half when `upper` is false and the hi half otherwise, sends the other half to its DPP partner
// (whose `upper` is the opposite) and combines what it keeps with what it receives.
template <int CTRL, int N>
__device__ __forceinline__ void minmax_step(const float* mn, const float* mx, bool upper, float* omn,
                                            float* omx) {
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const float kmn = upper ? mn[N + j] : mn[j], smn = upper ? mn[j] : mn[N + j];
    const float kmx = upper ? mx[N + j] : mx[j], smx = upper ? mx[j] : mx[N + j];
    const float rmn = dpp_f<CTRL>(smn), rmx = dpp_f<CTRL>(smx);
    omn[j] = rmn < kmn ? rmn : kmn;
    omx[j] = rmx > kmx ? rmx : kmx;
  }
}

// Min and max of each of 16 tokens over a 16-lane row, where every lane holds its own value of
// every token (mn[p], mx[p]): lane r of the row gets token r's. A butterfly: partners r^15
// (mirror), r^7 (half mirror), r^2 and r^1 each differ in the bit that decides which half of
// the remaining tokens a lane keeps, and the four steps together reach all 16 lanes. 15 lane
// exchanges per quantity instead of 64 for a reduction of every token.
__device__ __forceinline__ void row_minmax16(const float (&mn)[16], const float (&mx)[16], float& mn_r,
                                             float& mx_r) {
  const uint32_t r = threadIdx.x % 16;
  float a[8], b[8], c[4], d[4], e[2], f[2];
  minmax_step<kDppMirror, 8>(mn, mx, (r & 8) != 0, a, b);
  minmax_step<kDppHalfMirror, 4>(a, b, (r & 4) != 0, c, d);
  minmax_step<kDppXor2, 2>(c, d, (r & 2) != 0, e, f);
  minmax_step<kDppXor1, 1>(e, f, (r & 1) != 0, &mn_r, &mx_r);
}

// OR over aligned groups of L lanes (L a power of two <= 16).
template <uint32_t L>
__device__ __forceinline__ uint32_t group_or(uint32_t v) {
  if constexpr (L >= 2) v |= dpp_u<kDppXor1>(v);
  if constexpr (L >= 4) v |= dpp_u<kDppXor2>(v);
  if constexpr (L >= 8) v |= dpp_u<kDppHalfMirror>(v);
  if constexpr (L >= 16) v |= dpp_u<kDppMirror>(v);
  return v;
}

__device__ __forceinline__ const float* source_row(const RowSource& s, uint32_t unit, uint64_t i,
                                                   uint32_t R, uint32_t D) {
  uint64_t tok = s.offset + i;
  if (s.ring) tok %= R;
  return s.base + unit * s.stride_unit + tok * D;
}

// m = max(m, v) for a float v >= 0 kept as its bit pattern (device-scope atomic).
__device__ __forceinline__ void raise_to(uint32_t* m, float v) { atomicMax(m, __float_as_uint(v)); }

// Raise the running maxima m[0] (largest scale) and m[2] (largest |x|) of a unit's record
// (kMaxKeyScale / kMaxKeyAbs from a key record, kMaxValueScale / kMaxValueAbs from m = the
// record + 1) to the largest `scale` / `amax` of the workgroup.
__device__ __forceinline__ void raise_max(uint32_t* m, float scale, float amax) {
  __shared__ float red[2][kThreads / 64];
  for (int o = 32; o > 0; o >>= 1) {
    scale = fmaxf(scale, __shfl_xor(scale, o));
    amax = fmaxf(amax, __shfl_xor(amax, o));
  }
  if (threadIdx.x % 64 == 0) {
    red[0][threadIdx.x / 64] = scale;
    red[1][threadIdx.x / 64] = amax;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float a = red[0][0], b = red[1][0];
    for (int w = 1; w < kThreads / 64; ++w) {
      a = fmaxf(a, red[0][w]);
      b = fmaxf(b, red[1][w]);
    }
    raise_to(m, a);
    raise_to(m + 2, b);
  }
}

unsigned grid_for(uint64_t work, unsigned per_block = kThreads) {
  uint64_t b = (work + per_block - 1) / per_block;
  if (b > (1u << 20)) b = 1u << 20;  // grid-stride loops cover the rest
  if (b == 0) b = 1;
  return static_cast<unsigned>(b);
}

// ------------------------------------------------------------------ row copies

template <int VEC>
__global__ void __launch_bounds__(kThreads)
    k_copy_rows(RowSource src, float* dst, uint32_t R, uint32_t D, uint32_t units,
                uint32_t dst_slot, uint32_t count) {
  const uint32_t per_row = D / VEC;
  const uint64_t total = (uint64_t)units * count * per_row;
  for (uint64_t idx = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (uint64_t)gridDim.x * blockDim.x) {
    const uint32_t c = idx % per_row;
    const uint64_t r = idx / per_row;
    const uint32_t i = r % count;
    const uint32_t unit = r / count;
    const float* s = source_row(src, unit, i, R, D) + c * VEC;
    float* d = dst + ((uint64_t)unit * R + (dst_slot + i) % R) * D + c * VEC;
    if constexpr (VEC == 4) {
      *reinterpret_cast<float4*>(d) = *reinterpret_cast<const float4*>(s);
    } else {
      *d = *s;
    }
  }
}

// One decode token (see launch_decode_append): one workgroup per unit, thread d owns channel
// d. The value group min/max (src/quant.rs:349-375) reduces over the G lanes of a channel
// group by shuffles (G divides 64). Each channel's code word is read, OR-ed and written by
// its own thread (the words of a 64-token block fill across appends; later tokens' bits are
// still zero).
__global__ void __launch_bounds__(256)
    k_decode_append(CacheView c, const float* keys, const float* values, uint32_t kslot,
                    uint32_t vslot, uint32_t evict, uint64_t vq) {
  const Geometry& geo = c.geo;
  const uint32_t unit = blockIdx.x, d = threadIdx.x, D = geo.D, R = geo.R;
  c.kres[((uint64_t)unit * R + kslot) * D + d] = keys[(uint64_t)unit * D + d];
  const float v = values[(uint64_t)unit * D + d];
  float* slot = c.vring + ((uint64_t)unit * R + vslot) * D + d;
  if (evict) {
    const uint32_t G = geo.G, bits = geo.bits;
    const float levels = static_cast<float>(geo.levels());
    const float x = *slot;  // stream token vq, the oldest of the window
    float mn = x, mx = x;
    for (uint32_t o = 1; o < G; o <<= 1) {
      mn = fminf(mn, __shfl_xor(mn, o));
      mx = fmaxf(mx, __shfl_xor(mx, o));
    }
    const float fz = lane_group_first_zero(x, G);  // whole wave: the ballot needs every lane
    if (mn == 0.f) mn = fz;
    const float scale = scale_of(mx - mn, levels);
    const uint32_t code = quant_code(x, mn, scale, levels);
    const uint64_t tb = vq / kValueBlock;
    const uint32_t tt = static_cast<uint32_t>(vq % kValueBlock), ppw = geo.ppw(), vw = geo.vwords_per_channel();
    float2* params = reinterpret_cast<float2*>(c.vparams + unit * geo.vparams_unit());
    if (d % G == 0) params[(tb * geo.ncg() + d / G) * kValueBlock + tt] = make_float2(scale, mn);
    uint32_t* w = c.vcodes + unit * geo.vcodes_unit() + tb * D * vw + (uint64_t)d * vw + tt / ppw;
    *w = (tt % ppw == 0 ? 0u : *w) | (code << code_shift(bits, tt % ppw));
    // per-wave maxima of the scale and |x| (every lane holds its group's), one atomic each
    float sm = scale, am = fmaxf(fabsf(mn), fabsf(mx));
    for (int o = 32; o > 0; o >>= 1) {
      sm = fmaxf(sm, __shfl_xor(sm, o));
      am = fmaxf(am, __shfl_xor(am, o));
    }
    if (d % 64 == 0) {
      atomicMax(max_slot(c, unit, 0) + kMaxValueScale, __float_as_uint(sm));
      atomicMax(max_slot(c, unit, 0) + kMaxValueAbs, __float_as_uint(am));
    }
  }
  *slot = v;
}

// Workgroup (unit, kind): kind 0 scans the key residual rows, kind 1 the value window rows.
__global__ void __launch_bounds__(kThreads)
    k_raise_row_max(CacheView c, uint32_t kres, uint32_t vres, uint32_t vhead) {
  const Geometry& geo = c.geo;
  const uint32_t unit = blockIdx.x / 2, kind = blockIdx.x % 2, D = geo.D, R = geo.R;
  const uint32_t rows = kind == 0 ? kres : vres;
  const float* base = (kind == 0 ? c.kres : c.vring) + (uint64_t)unit * R * D;
  float m = 0.f;
  for (uint32_t i = threadIdx.x; i < rows * D; i += blockDim.x) {
    const uint32_t r = i / D, d = i % D;
    const uint32_t slot = kind == 0 ? r : (vhead + r) % R;
    m = fmaxf(m, fabsf(base[(uint64_t)slot * D + d]));
  }
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  if (threadIdx.x % 64 == 0) atomicMax(max_slot(c, unit, 0) + kMaxKeyAbs + kind, __float_as_uint(m));
}

// Rows are staged through LDS as floats [rows][D+1] (the odd stride spreads a column over the
// banks) by coalesced reads, float4 when `vec4`; at most kStageFloats floats per pass.
constexpr uint32_t kStageFloats = 8704;  // 34 KiB

__device__ __forceinline__ void stage_row(const float* src, float* dst, uint32_t D, bool vec4,
                                          uint32_t part, uint32_t parts) {
  if (vec4) {
    for (uint32_t c4 = part; c4 < D / 4; c4 += parts) {
      typedef float f4v_ __attribute__((ext_vector_type(4)));
      const f4v_ v = __builtin_nontemporal_load(reinterpret_cast<const f4v_*>(src) + c4);
      dst[4 * c4] = v.x;
      dst[4 * c4 + 1] = v.y;
      dst[4 * c4 + 2] = v.z;
      dst[4 * c4 + 3] = v.w;
    }
  } else {
    for (uint32_t c = part; c < D; c += parts) dst[c] = __builtin_nontemporal_load(src + c);
  }
}

// ------------------------------------------------------------------ keys (native layout)
// One workgroup per (unit, group): per-channel min/max over the group's G tokens
// (src/quant.rs:296-306), (scale, zero) per channel (:307-311), codes for every token
// (:312-323), then token-major words. The G x D block is staged in LDS in one coalesced pass
// when it fits (`staged`), else read from global memory directly.
__global__ void __launch_bounds__(kThreads)
    k_quant_keys(CacheView c, RowSource src, uint64_t g0, uint32_t ngroups, uint32_t staged,
                 uint32_t vec4) {
  extern __shared__ uint8_t smem[];
  const Geometry& geo = c.geo;
  const uint32_t G = geo.G, D = geo.D, bits = geo.bits;
  uint8_t* codes_lds = smem;                                                // [G][D]
  float* xs = reinterpret_cast<float*>(smem + ((size_t)G * D + 15) / 16 * 16);  // [G][D+1]
  const float levels = static_cast<float>(geo.levels());
  const uint32_t unit = blockIdx.x / ngroups;
  const uint32_t g = blockIdx.x % ngroups;
  const float* rows = src.base + unit * src.stride_unit + (src.offset + (uint64_t)g * G) * D;
  float2* params = reinterpret_cast<float2*>(c.kparams + unit * geo.kparams_unit() + (g0 + g) * D * 2);
  if (staged) {
    // a wave per row at a time, all rows' loads in flight across the workgroup
    const uint32_t lanes = 64, waves = blockDim.x / 64;
    for (uint32_t t = threadIdx.x / lanes; t < G; t += waves)
      stage_row(rows + (uint64_t)t * D, xs + t * (D + 1), D, vec4 != 0, threadIdx.x % lanes, lanes);
    __syncthreads();
  }
  float smax = 0.f, amax = 0.f;
  for (uint32_t d = threadIdx.x; d < D; d += blockDim.x) {
    float mn = INFINITY, mx = -INFINITY;
    for (uint32_t t = 0; t < G; ++t) {
      const float x = staged ? xs[t * (D + 1) + d] : rows[(uint64_t)t * D + d];
      mn = x < mn ? x : mn;  // keeps the first of equal minima (the first zero)
      mx = fmaxf(mx, x);
    }
    const float zero = mn;
    const float scale = scale_of(mx - zero, levels);
    smax = fmaxf(smax, scale);
    amax = fmaxf(amax, fmaxf(fabsf(mn), fabsf(mx)));
    params[d] = make_float2(scale, zero);
    for (uint32_t t = 0; t < G; ++t) {
      const float x = staged ? xs[t * (D + 1) + d] : rows[(uint64_t)t * D + d];
      codes_lds[t * D + d] = static_cast<uint8_t>(quant_code(x, zero, scale, levels));
    }
  }
  raise_max(max_slot(c, unit, blockIdx.x) + kMaxKeyScale, smax, amax);  // includes the barrier before the packing below
  const uint32_t ppw = geo.ppw();
  const uint32_t kw = geo.kwords_per_token();
  uint32_t* words = c.kcodes + unit * geo.kcodes_unit() + (g0 + g) * G * kw;
  for (uint32_t w = threadIdx.x; w < G * kw; w += blockDim.x) {
    const uint32_t t = w / kw, j = w % kw;
    const uint8_t* cc = codes_lds + t * D + j * ppw;
    uint32_t word = 0;
    for (uint32_t i = 0; i < ppw; ++i) word |= static_cast<uint32_t>(cc[i]) << code_shift(bits, i);
    words[w] = word;
  }
}

// ------------------------------------------------------------------ values (native layout)
// One workgroup per (unit, 64-token block touched). Phase 1, per batch of TB tokens: the rows
// are staged in LDS (coalesced), then one thread per (token, channel group) computes min/max,
// (scale, zero) and codes (src/quant.rs:349-375). Phase 2: one thread per channel-major word;
// words that already hold earlier tokens of the block are read, OR-ed and written back
// (blocks fill across appends).
__global__ void __launch_bounds__(kThreads)
    k_quant_values(CacheView c, RowSource ring, uint32_t n_ring, RowSource in, uint64_t vq0,
                   uint64_t n, uint64_t blk0, uint32_t nblk, uint32_t TB, uint32_t vec4) {
  extern __shared__ uint8_t smem[];
  const Geometry& geo = c.geo;
  const uint32_t G = geo.G, D = geo.D, bits = geo.bits, R = geo.R, ncg = geo.ncg();
  uint8_t* codes_lds = smem;                                                        // [64][D]
  float* xs = reinterpret_cast<float*>(smem + ((size_t)kValueBlock * D + 15) / 16 * 16);  // [TB][D+1]
  const float levels = static_cast<float>(geo.levels());
  const uint32_t unit = blockIdx.x / nblk;
  const uint64_t tb = blk0 + blockIdx.x % nblk;
  const uint64_t t_lo = vq0 > tb * kValueBlock ? vq0 : tb * kValueBlock;
  const uint64_t t_end = vq0 + n;
  const uint64_t t_hi = t_end < (tb + 1) * kValueBlock ? t_end : (tb + 1) * kValueBlock;
  const uint32_t ntok = static_cast<uint32_t>(t_hi - t_lo);
  float2* params = reinterpret_cast<float2*>(c.vparams + unit * geo.vparams_unit());
  float smax = 0.f, amax = 0.f;
  const uint32_t lanes = 64, waves = blockDim.x / 64;
  for (uint32_t k0 = 0; k0 < ntok; k0 += TB) {
    const uint32_t nb = ntok - k0 < TB ? ntok - k0 : TB;
    for (uint32_t r = threadIdx.x / lanes; r < nb; r += waves) {
      const uint64_t i = t_lo + k0 + r - vq0;
      const float* row = i < n_ring ? source_row(ring, unit, i, R, D) : source_row(in, unit, i - n_ring, R, D);
      stage_row(row, xs + r * (D + 1), D, vec4 != 0, threadIdx.x % lanes, lanes);
    }
    __syncthreads();
    // token fastest, so neighbouring threads read neighbouring rows (distinct banks)
    for (uint32_t p = threadIdx.x; p < nb * ncg; p += blockDim.x) {
      const uint32_t r = p % nb, cg = p / nb;
      const float* grp = xs + r * (D + 1) + cg * G;
      float mn = INFINITY, mx = -INFINITY;
      for (uint32_t e = 0; e < G; ++e) {
        mn = grp[e] < mn ? grp[e] : mn;  // keeps the first of equal minima (the first zero)
        mx = fmaxf(mx, grp[e]);
      }
      const float scale = scale_of(mx - mn, levels);
      smax = fmaxf(smax, scale);
      amax = fmaxf(amax, fmaxf(fabsf(mn), fabsf(mx)));
      const uint64_t t = t_lo + k0 + r;
      const uint32_t tt = static_cast<uint32_t>(t % kValueBlock);
      params[(tb * ncg + cg) * kValueBlock + tt] = make_float2(scale, mn);
      uint8_t* dst = codes_lds + tt * D + cg * G;
      for (uint32_t e = 0; e < G; ++e) dst[e] = static_cast<uint8_t>(quant_code(grp[e], mn, scale, levels));
    }
    __syncthreads();  // the staging buffer is refilled by the next batch
  }
  raise_max(max_slot(c, unit, blockIdx.x) + kMaxValueScale, smax, amax);  // includes the barrier before the packing below
  const uint32_t ppw = geo.ppw();
  const uint32_t vw = geo.vwords_per_channel();
  const uint32_t w_lo = static_cast<uint32_t>(t_lo % kValueBlock) / ppw;
  const uint32_t w_hi = static_cast<uint32_t>((t_hi - 1) % kValueBlock) / ppw + 1;
  const uint32_t nw = w_hi - w_lo;
  uint32_t* base = c.vcodes + unit * geo.vcodes_unit() + tb * D * vw;
  for (uint32_t idx = threadIdx.x; idx < D * nw; idx += blockDim.x) {
    const uint32_t d = idx / nw, w = w_lo + idx % nw;
    uint32_t word = 0;
    bool keep_old = false;
    for (uint32_t i = 0; i < ppw; ++i) {
      const uint64_t t = tb * kValueBlock + w * ppw + i;
      if (t >= t_lo && t < t_hi) {
        word |= static_cast<uint32_t>(codes_lds[(t % kValueBlock) * D + d]) << code_shift(bits, i);
      } else if (t < t_lo) {
        keep_old = true;
      }
    }
    uint32_t* dst = base + (uint64_t)d * vw + w;
    if (keep_old) word |= *dst;
    *dst = word;
  }
}

// ------------------------------------------------------------------ wave-per-item fast paths
// For head_dim = 64*CPL (CPL = 1, 2, 4): lane l of a wave holds channels CPL*l .. +CPL-1 of a
// row, so every row is one coalesced wave load and the quantization runs in registers; only
// the codes go through LDS for the packing.

// The rows are read once: non-temporal loads (measured 12-17% faster quantize at the
// benchmark shapes than cached loads).
typedef float f2v __attribute__((ext_vector_type(2)));
typedef float f4v __attribute__((ext_vector_type(4)));
template <int CPL>
__device__ __forceinline__ void load_lane(const float* row, uint32_t lane, float (&x)[CPL]) {
  if constexpr (CPL == 4) {
    const f4v v = __builtin_nontemporal_load(reinterpret_cast<const f4v*>(row) + lane);
    x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
  } else if constexpr (CPL == 2) {
    const f2v v = __builtin_nontemporal_load(reinterpret_cast<const f2v*>(row) + lane);
    x[0] = v.x; x[1] = v.y;
  } else {
    x[0] = __builtin_nontemporal_load(row + lane);
  }
}

__device__ __forceinline__ void wave_raise_max(uint32_t* m, float scale, float amax) {
  for (int o = 32; o > 0; o >>= 1) {
    scale = fmaxf(scale, __shfl_xor(scale, o));
    amax = fmaxf(amax, __shfl_xor(amax, o));
  }
  if (threadIdx.x % 64 == 0) {
    raise_to(m, scale);
    raise_to(m + 2, amax);
  }
}

// Keys: workgroup (unit, span) takes groups span*kKeySpan .. +kKeySpan-1 of the unit, wave w
// those = w (mod 4); the lane keeps its channels of a group's GG rows in registers for the
// per-channel min/max (src/quant.rs:296-311). Codes are packed in registers: the LPW lanes
// whose channels share a token-major word OR their parts together (DPP), lane m of the group
// keeps the words of tokens t = m (mod LPW), and each store writes 64 consecutive words. The
// unit's running maxima are raised once per workgroup, in the maxima record its index selects.
constexpr uint32_t kKeySpan = 4;  // one group per wave
template <int BITS, int CPL, int GG>
__global__ void __launch_bounds__(kThreads)
    k_quant_keys_wave(CacheView c, RowSource src, uint64_t g0, uint32_t ngroups, uint32_t spans) {
  constexpr uint32_t D = 64 * CPL, PPW = 32 / BITS;
  constexpr uint32_t LPW = PPW / CPL;   // lanes per code word
  constexpr uint32_t KW = D / PPW;      // words per token (= 64 / LPW)
  constexpr uint32_t NS = GG / LPW;     // words kept per lane
  constexpr uint32_t kLevels = (1u << BITS) - 1u;
  constexpr float levels = static_cast<float>(kLevels);
  const Geometry& geo = c.geo;
  const uint32_t lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  const uint32_t unit = blockIdx.x / spans;
  const uint32_t g_end = std::min(ngroups, (blockIdx.x % spans + 1) * kKeySpan);
  float smax = 0.f, amax = 0.f;
  for (uint32_t g = (blockIdx.x % spans) * kKeySpan + wave; g < g_end; g += 4) {
    const float* rows = src.base + unit * src.stride_unit + (src.offset + (uint64_t)g * GG) * D;
    float x[GG][CPL];
#pragma unroll
    for (int t = 0; t < GG; ++t) load_lane<CPL>(rows + (uint64_t)t * D, lane, x[t]);
    float2 sz[CPL];
    float inv[CPL];
    uint32_t sh[CPL];
    float mns[CPL], mxs[CPL];
    bool zero_min = false;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      float mn = INFINITY, mx = -INFINITY;
#pragma unroll
      for (int t = 0; t < GG; ++t) {
        mn = fminf(mn, x[t][j]);
        mx = fmaxf(mx, x[t][j]);
      }
      mns[j] = mn;
      mxs[j] = mx;
      zero_min |= mn == 0.f;
    }
    if (__ballot(zero_min)) {  // rare, and wave-uniform: a zero minimum takes its first zero's sign
#pragma unroll
      for (int j = 0; j < CPL; ++j)
        if (mns[j] == 0.f) mns[j] = first_zero(rows + CPL * lane + j, D, GG);
    }
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const float mn = mns[j], mx = mxs[j];
      sz[j] = make_float2(scale_of(mx - mn, levels), mn);
      inv[j] = quant_inv(sz[j].x);
      sh[j] = code_shift(BITS, (CPL * lane + j) % PPW);
      smax = fmaxf(smax, sz[j].x);
      amax = fmaxf(amax, fmaxf(fabsf(mn), fabsf(mx)));
    }
    float2* params = reinterpret_cast<float2*>(c.kparams + unit * geo.kparams_unit() + (g0 + g) * D * 2);
#pragma unroll
    for (int j = 0; j < CPL; ++j) params[CPL * lane + j] = sz[j];
    const uint32_t m = lane % LPW;
    uint32_t keep[NS];
#pragma unroll
    for (int t = 0; t < GG; ++t) {
      uint32_t part = 0;
#pragma unroll
      for (int j = 0; j < CPL; ++j) part |= quant_code_fast(x[t][j], sz[j].y, sz[j].x, inv[j], kLevels) << sh[j];
      part = group_or<LPW>(part);
      if (t % LPW == 0) keep[t / LPW] = part;
      else if (m == t % LPW) keep[t / LPW] = part;
    }
    uint32_t* words = c.kcodes + unit * geo.kcodes_unit() + (g0 + g) * GG * KW;
#pragma unroll
    for (int s2 = 0; s2 < (int)NS; ++s2) words[(s2 * LPW + m) * KW + lane / LPW] = keep[s2];
  }
  raise_max(max_slot(c, unit, blockIdx.x) + kMaxKeyScale, smax, amax);
}

// Values: workgroup (unit, span) takes the unit's 64-token blocks span*kValueSpan .. +kValueSpan-1
// of this call; in each, wave w takes the block's tokens 16w .. 16w+15 that lie in the call's
// range. A lane holds channels CPL*lane .. +CPL-1 of each row; the group min/max
// (src/quant.rs:349-375) reduces over the G/CPL lanes of a channel group (DPP), and the lane
// packs its channels' codes of the 16 tokens into their channel-major words in registers
// (16/PPW words per channel). The four waves' words meet in LDS (two buffers, one barrier per
// block) so each block's words are stored contiguously; words that already hold earlier tokens
// of the block are read and OR-ed (blocks fill across appends). The unit's running maxima are
// raised once per workgroup, in the maxima record its index selects.
constexpr uint32_t kValueSpan = 1;  // one block per workgroup
template <int BITS, int CPL, int GG>
__global__ void __launch_bounds__(kThreads)
    k_quant_values_wave(CacheView c, RowSource ring, uint32_t n_ring, RowSource in, uint64_t vq0,
                        uint64_t n, uint64_t blk0, uint32_t nblk, uint32_t spans) {
  constexpr uint32_t D = 64 * CPL, PPW = 32 / BITS, WPW = 16 / PPW;
  constexpr uint32_t kLevels = (1u << BITS) - 1u;
  constexpr float levels = static_cast<float>(kLevels);
  constexpr uint32_t L = GG / CPL;  // lanes per channel group
  constexpr uint32_t VW = kValueBlock / PPW, VWP = VW + 1;  // words per channel (LDS row padded)
  __shared__ uint32_t words_lds[2][D * VWP];
  const Geometry& geo = c.geo;
  const uint32_t R = geo.R, ncg = geo.ncg();
  const uint32_t lane = threadIdx.x % 64;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);  // wave-uniform
  const uint32_t unit = blockIdx.x / spans;
  const uint32_t b_first = (blockIdx.x % spans) * kValueSpan;
  const uint32_t b_end = std::min(nblk, b_first + kValueSpan);
  float2* params = reinterpret_cast<float2*>(c.vparams + unit * geo.vparams_unit());
  const uint32_t cg = CPL * lane / GG;
  float smax = 0.f, amax = 0.f;
  for (uint32_t bi = b_first; bi < b_end; ++bi) {
    const uint64_t tb = blk0 + bi;
    uint32_t* wl = words_lds[bi % 2];
    const uint64_t t0 = tb * kValueBlock + 16 * wave;  // first token of the wave's slot
    const uint64_t t_lo = vq0 > t0 ? vq0 : t0;
    const uint64_t t_hi = vq0 + n < t0 + 16 ? vq0 + n : t0 + 16;
    if (t_lo < t_hi) {
      float x[16][CPL];
      // token t0 + p reads a valid row: t clamped to [t_lo, t_hi)
      const uint32_t p_lo = static_cast<uint32_t>(t_lo - t0), p_hi = static_cast<uint32_t>(t_hi - 1 - t0);
      if (t_lo - vq0 >= n_ring && !in.ring) {
        // every row from the (linear) input: consecutive rows from the slot's first valid one
        const float* row0 = in.base + unit * in.stride_unit + (in.offset + (t_lo - vq0 - n_ring)) * D;
#pragma unroll
        for (int p = 0; p < 16; ++p) {
          const uint32_t pc = (uint32_t)p < p_lo ? p_lo : (uint32_t)p > p_hi ? p_hi : (uint32_t)p;
          load_lane<CPL>(row0 + (pc - p_lo) * D, lane, x[p]);
        }
      } else {
#pragma unroll
        for (int p = 0; p < 16; ++p) {
          const uint32_t pc = (uint32_t)p < p_lo ? p_lo : (uint32_t)p > p_hi ? p_hi : (uint32_t)p;
          const uint64_t i = t0 + pc - vq0;
          const float* row = i < n_ring ? source_row(ring, unit, i, R, D) : source_row(in, unit, i - n_ring, R, D);
          load_lane<CPL>(row, lane, x[p]);
        }
      }
      uint32_t word[CPL][WPW];
#pragma unroll
      for (int j = 0; j < CPL; ++j)
#pragma unroll
        for (int k = 0; k < (int)WPW; ++k) word[j][k] = 0;
      if constexpr (L == 16) {
        // A channel group is a DPP row of 16 lanes and the wave has 16 rows: the group's
        // min/max of row r ends in lane r (row_minmax16), which divides for row r once (one
        // division for the 16 rows) and stores row r's (scale, zero) (16 consecutive pairs per
        // group); row_newbcast hands each row's zero, scale and reciprocal to the group's lanes.
        float pmn[16], pmx[16];
#pragma unroll
        for (int p = 0; p < 16; ++p) {
          pmn[p] = pmx[p] = x[p][0];
#pragma unroll
          for (int j = 1; j < CPL; ++j) minmax_with(pmn[p], pmx[p], x[p][j], x[p][j]);
        }
        float mn_r, mx_r;
        row_minmax16(pmn, pmx, mn_r, mx_r);
        const uint32_t r = lane % 16;
        if (__ballot(mn_r == 0.f)) {  // rare, and wave-uniform: row r's first zero gives the sign
          if (mn_r == 0.f) {
            const uint64_t i = t0 + (r < p_lo ? p_lo : r > p_hi ? p_hi : r) - vq0;
            const float* row = i < n_ring ? source_row(ring, unit, i, R, D) : source_row(in, unit, i - n_ring, R, D);
            mn_r = first_zero(row + cg * GG, 1, GG);
          }
        }
        const float scale_r = scale_of(mx_r - mn_r, levels);
        const float inv_r = quant_inv(scale_r);
        if (t0 + r >= t_lo && t0 + r < t_hi) {
          smax = fmaxf(smax, scale_r);
          amax = fmaxf(amax, fmaxf(fabsf(mn_r), fabsf(mx_r)));
          params[(tb * ncg + cg) * kValueBlock + 16 * wave + r] = make_float2(scale_r, mn_r);
        }
#pragma unroll
        for (int p = 0; p < 16; ++p) {
          const bool valid = t0 + p >= t_lo && t0 + p < t_hi;
          const float scale = row_bcast(scale_r, p), inv = row_bcast(inv_r, p);
          const float zero = row_bcast(mn_r, p);
#pragma unroll
          for (int j = 0; j < CPL; ++j) {
            const uint32_t code = quant_code_fast(x[p][j], zero, scale, inv, kLevels);
            word[j][p / PPW] |= (valid ? code : 0u) << code_shift(BITS, p % PPW);
          }
        }
      } else {
#pragma unroll
        for (int p = 0; p < 16; ++p) {
          const bool valid = t0 + p >= t_lo && t0 + p < t_hi;
          float mn = x[p][0], mx = x[p][0];
#pragma unroll
          for (int j = 1; j < CPL; ++j) minmax_with(mn, mx, x[p][j], x[p][j]);
          group_minmax<L>(mn, mx);
          if (__ballot(mn == 0.f)) {  // rare, and wave-uniform: row p's first zero gives the sign
            const uint64_t i = t0 + ((uint32_t)p < p_lo ? p_lo : (uint32_t)p > p_hi ? p_hi : (uint32_t)p) - vq0;
            const float* row = i < n_ring ? source_row(ring, unit, i, R, D) : source_row(in, unit, i - n_ring, R, D);
            if (mn == 0.f) mn = first_zero(row + cg * GG, 1, GG);
          }
          const float scale = scale_of(mx - mn, levels);
          const float inv = quant_inv(scale);
          if (valid) {
            smax = fmaxf(smax, scale);
            amax = fmaxf(amax, fmaxf(fabsf(mn), fabsf(mx)));
            if (lane % L == 0) params[(tb * ncg + cg) * kValueBlock + 16 * wave + p] = make_float2(scale, mn);
          }
#pragma unroll
          for (int j = 0; j < CPL; ++j) {
            const uint32_t code = quant_code_fast(x[p][j], mn, scale, inv, kLevels);
            word[j][p / PPW] |= (valid ? code : 0u) << code_shift(BITS, p % PPW);
          }
        }
      }
#pragma unroll
      for (int j = 0; j < CPL; ++j)
#pragma unroll
        for (int k = 0; k < (int)WPW; ++k) wl[(CPL * lane + j) * VWP + 16 * wave / PPW + k] = word[j][k];
    }
    __syncthreads();  // the block's words are in wl (the other buffer is free for the next block)
    // the block's words with a token of this call: [b_lo, b_hi) is the call's range in the block
    const uint64_t blk = tb * kValueBlock;
    const uint64_t b_lo = vq0 > blk ? vq0 : blk;
    const uint64_t b_hi = vq0 + n < blk + kValueBlock ? vq0 + n : blk + kValueBlock;
    uint32_t* base = c.vcodes + unit * geo.vcodes_unit() + tb * D * VW;
    for (uint32_t idx = threadIdx.x; idx < D * VW; idx += blockDim.x) {
      const uint32_t d = idx / VW, wi = idx % VW;
      const uint64_t w0 = blk + wi * PPW;  // first token of word wi
      if (w0 + PPW <= b_lo || w0 >= b_hi) continue;
      const uint32_t v = wl[d * VWP + wi];
      base[idx] = w0 < b_lo ? (v | base[idx]) : v;
    }
  }
  raise_max(max_slot(c, unit, blockIdx.x) + kMaxValueScale, smax, amax);
}

// ------------------------------------------------------------------ export to reference order

// Swap mask of a block-transpose round: the low s-element half of every 2s-element run of a
// word of 32/bits elements.
constexpr uint32_t swap_mask(uint32_t bits, uint32_t s) {
  uint32_t m = 0;
  for (uint32_t e = 0; e < 32 / bits; ++e)
    if ((e / s) % 2 == 0) m |= ((1u << bits) - 1u) << (bits * e);
  return m;
}

// Transpose of a PPW x PPW block of codes held in PPW native words: word t holds row t, its
// element i at bit code_shift(BITS, i). Afterwards word code_shift(BITS, i) / BITS holds
// column i with row t at bit BITS*t, the reference's order (first element in the low bits).
// log2(PPW) rounds: in the round of half-size s, the upper s-element half of each 2s-element
// run of row t (t & s == 0) trades places with the lower half of row t + s. A native word's
// elements sit at a permutation of the element slots, so the rounds move whole columns and
// only the output word that receives each column changes.
template <int BITS>
__device__ __forceinline__ void transpose_codes(uint32_t (&w)[32 / BITS]) {
  constexpr int N = 32 / BITS;
#pragma unroll
  for (int s = N / 2; s >= 1; s /= 2) {
    const uint32_t m = swap_mask(BITS, s);
#pragma unroll
    for (int t = 0; t < N; ++t) {
      if (t & s) continue;
      const uint32_t x = ((w[t] >> (BITS * s)) ^ w[t + s]) & m;
      w[t + s] ^= x;
      w[t] ^= x << (BITS * s);
    }
  }
}

// Key words (g*D + d)*ipc + w hold tokens g*G + w*ppw + i of channel d (src/quant.rs:312-323).
// Grid (group slices, units): a workgroup stages its `per` groups' native words in LDS
// (coalesced reads, one barrier); each thread then transposes one ppw x ppw block (ppw tokens
// of one native word of channels) in registers and puts its ppw output words in a second LDS
// buffer (`stage_out`; else straight to memory), which is written out with coalesced stores.
constexpr uint32_t kExportGroups = 8;        // groups per workgroup, at most
constexpr uint32_t kExportLdsWords = 16384;  // staging words per workgroup, at most (64 KB)
template <int BITS>
__global__ void __launch_bounds__(kThreads)
    k_export_keys(CacheView c, uint64_t kq, uint32_t per, uint32_t stage_out, uint32_t* out) {
  constexpr uint32_t PPW = 32 / BITS;
  // [per][kw][G + 4]: native word (token t, channel word k) at k * (G + 4) + t, so that the
  // PPW tokens of a block are 16-byte reads (rows 16-byte aligned, 4 banks apart); then
  // [per][n] output words when staged
  extern __shared__ uint32_t words[];
  const Geometry& geo = c.geo;
  const uint32_t G = geo.G, kw = geo.kwords_per_token(), row = G + 4;
  const uint32_t ipc = G / PPW, n = G * kw, np = kw * row;  // words per group, both orders
  const uint64_t ngroups = kq / G;
  const uint64_t g0 = (uint64_t)blockIdx.x * per;
  const uint32_t ng = static_cast<uint32_t>(std::min<uint64_t>(per, ngroups - g0));
  uint32_t* staged = words + per * np;
  for (uint32_t unit = blockIdx.y; unit < geo.units; unit += gridDim.y) {
    const uint32_t* src = c.kcodes + unit * geo.kcodes_unit() + g0 * n;
    uint32_t* dst = out + (uint64_t)unit * ngroups * n + g0 * n;
    for (uint32_t i = threadIdx.x; i < ng * n; i += blockDim.x) {
      const uint32_t gg = i / n, r = i % n;
      words[gg * np + (r % kw) * row + r / kw] = src[i];
    }
    __syncthreads();
    // block (group gg, channel word k, token run tb): channels k*PPW + i, tokens tb*PPW + t
    for (uint32_t task = threadIdx.x; task < ng * kw * ipc; task += blockDim.x) {
      const uint32_t gg = task / (kw * ipc), r = task % (kw * ipc), k = r / ipc, tb = r % ipc;
      const uint4* tw = reinterpret_cast<const uint4*>(words + gg * np + k * row + tb * PPW);
      uint32_t w[PPW];
#pragma unroll
      for (uint32_t q = 0; q < PPW / 4; ++q) {
        const uint4 x = tw[q];
        w[4 * q] = x.x;
        w[4 * q + 1] = x.y;
        w[4 * q + 2] = x.z;
        w[4 * q + 3] = x.w;
      }
      transpose_codes<BITS>(w);
#pragma unroll
      for (uint32_t i = 0; i < PPW; ++i) {
        const uint32_t o = gg * n + (k * PPW + i) * ipc + tb;
        const uint32_t v = w[code_shift(BITS, i) / BITS];
        if (stage_out) staged[o] = v;
        else dst[o] = v;
      }
    }
    if (stage_out) {
      __syncthreads();
      for (uint32_t i = threadIdx.x; i < ng * n; i += blockDim.x) dst[i] = staged[i];
    }
    __syncthreads();  // the staging buffers are refilled for the next unit
  }
}

// Value words (t*(D/G) + cg)*ipg + w = t*(D/ppw) + j hold channels j*ppw + i of token t
// (src/quant.rs:362-372); params (t*(D/G) + cg)*2 (src/quant.rs:360-361). Grid (block slices,
// units): a workgroup stages its `per` 64-token blocks' native words in LDS; each thread
// transposes one ppw x ppw block (ppw channels of one native word of tokens) in registers into
// ppw output words, staged for coalesced stores as the key export does, and the (scale, zero)
// pairs are copied in token order.
constexpr uint32_t kExportBlocks = 4;  // 64-token blocks per workgroup, at most
template <int BITS>
__global__ void __launch_bounds__(kThreads)
    k_export_values(CacheView c, uint64_t vq, uint32_t per, uint32_t stage_out, uint32_t* out_codes,
                    float* out_params) {
  constexpr uint32_t PPW = 32 / BITS, VW = kValueBlock / PPW;
  // [per][VW][D + 4]: native word (channel c, word w) at w * (D + 4) + c, so that the PPW
  // channels of a block are 16-byte reads; then [per][64][D / PPW] output words when staged
  extern __shared__ uint32_t words[];
  const Geometry& geo = c.geo;
  const uint32_t D = geo.D, ncg = geo.ncg(), wpt = D / PPW, n = D * VW, row = D + 4, np = VW * row;
  const uint64_t nblk = (vq + kValueBlock - 1) / kValueBlock;
  const uint64_t b0 = (uint64_t)blockIdx.x * per;
  const uint32_t nb = static_cast<uint32_t>(std::min<uint64_t>(per, nblk - b0));
  // tokens of this workgroup's blocks (the last block of the stream may be partial)
  const uint32_t ntok = static_cast<uint32_t>(std::min<uint64_t>((uint64_t)nb * kValueBlock, vq - b0 * kValueBlock));
  uint32_t* staged = words + per * np;
  for (uint32_t unit = blockIdx.y; unit < geo.units; unit += gridDim.y) {
    const uint32_t* src = c.vcodes + unit * geo.vcodes_unit() + b0 * n;
    const float2* prm = reinterpret_cast<const float2*>(c.vparams + unit * geo.vparams_unit()) + b0 * ncg * kValueBlock;
    uint32_t* dst = out_codes + (uint64_t)unit * vq * wpt + b0 * kValueBlock * wpt;
    for (uint32_t i = threadIdx.x; i < nb * n; i += blockDim.x) {
      const uint32_t bb = i / n, r = i % n;  // r = channel * VW + word
      words[bb * np + (r % VW) * row + r / VW] = src[i];
    }
    __syncthreads();
    // block (block bb, channel run j, word w): channels j*PPW + t, tokens w*PPW + i
    for (uint32_t task = threadIdx.x; task < nb * wpt * VW; task += blockDim.x) {
      const uint32_t bb = task / (wpt * VW), r = task % (wpt * VW), j = r / VW, wd = r % VW;
      const uint4* tw = reinterpret_cast<const uint4*>(words + bb * np + wd * row + j * PPW);
      uint32_t w[PPW];
#pragma unroll
      for (uint32_t q = 0; q < PPW / 4; ++q) {
        const uint4 x = tw[q];
        w[4 * q] = x.x;
        w[4 * q + 1] = x.y;
        w[4 * q + 2] = x.z;
        w[4 * q + 3] = x.w;
      }
      transpose_codes<BITS>(w);
#pragma unroll
      for (uint32_t i = 0; i < PPW; ++i) {
        const uint32_t tk = bb * kValueBlock + wd * PPW + i;  // token within the workgroup's blocks
        const uint32_t v = w[code_shift(BITS, i) / BITS];
        if (stage_out) staged[tk * wpt + j] = v;
        else if (tk < ntok) dst[tk * wpt + j] = v;
      }
    }
    if (stage_out) {
      __syncthreads();
      for (uint32_t o = threadIdx.x; o < ntok * wpt; o += blockDim.x) dst[o] = staged[o];
    }
    if (out_params != nullptr) {
      float2* dpar = reinterpret_cast<float2*>(out_params) + ((uint64_t)unit * vq + b0 * kValueBlock) * ncg;
      for (uint32_t o = threadIdx.x; o < ntok * ncg; o += blockDim.x) {
        const uint32_t tk = o / ncg, cg = o % ncg, bb = tk / kValueBlock, tt = tk % kValueBlock;
        dpar[o] = prm[((uint64_t)bb * ncg + cg) * kValueBlock + tt];
      }
    }
    __syncthreads();  // the staging buffers are refilled for the next unit
  }
}

// ------------------------------------------------------------------ dense reconstruction

// KiviCache::dequantize (src/cache.rs:282-325): packed tokens as fma(code, scale, zero)
// (src/quant.rs:406, 443), residual tokens copied. A workgroup takes one 64-token block of a
// unit at a time and stages everything the block's packed tokens read in LDS with coalesced
// loads: the value words as [word][channel] rows padded by 4 words (the four channels of a
// float4 are one 16-byte read, and the transposing writes spread over the banks), the value
// (scale, zero) pairs, the key words as stored and the (scale, zero) pairs of the key groups
// the block touches. A thread then writes float4 runs of consecutive channels (D % 4 == 0) of
// keys and values from LDS only.
struct DequantLds {
  uint32_t vrow, vwords, vparams, kwords, kgroups, kparams, total;  // offsets and sizes in words
};
__host__ __device__ inline DequantLds dequant_lds(const Geometry& g) {
  DequantLds l;
  l.vrow = g.D + 4;
  l.vwords = 0;
  l.vparams = g.vwords_per_channel() * l.vrow;
  l.kwords = l.vparams + 2 * g.ncg() * kValueBlock;
  l.kgroups = (kValueBlock + g.G - 1) / g.G + 1;  // groups a run of 64 tokens can touch
  l.kparams = l.kwords + kValueBlock * g.kwords_per_token();
  l.total = l.kparams + 2 * l.kgroups * g.D;
  return l;
}
__global__ void __launch_bounds__(kThreads)
    k_dequant_cache(CacheView c, SeqState s, uint64_t seq, float* keys, float* values) {
  extern __shared__ uint32_t stage[];
  const Geometry& geo = c.geo;
  const DequantLds L = dequant_lds(geo);
  const uint32_t D = geo.D, G = geo.G, R = geo.R, bits = geo.bits, ppw = geo.ppw();
  const uint32_t kw = geo.kwords_per_token(), vw = geo.vwords_per_channel(), ncg = geo.ncg();
  const uint32_t mask = geo.levels();
  const uint32_t q4 = D / 4;
  uint32_t* svw = stage + L.vwords;
  float2* svp = reinterpret_cast<float2*>(stage + L.vparams);
  uint32_t* skw = stage + L.kwords;
  float2* skp = reinterpret_cast<float2*>(stage + L.kparams);
  const uint64_t nblk = (seq + kValueBlock - 1) / kValueBlock;
  const uint64_t total = nblk * geo.units;
  for (uint64_t job = blockIdx.x; job < total; job += gridDim.x) {
    const uint32_t unit = static_cast<uint32_t>(job / nblk);
    const uint64_t tb = job % nblk;
    const uint64_t t0 = tb * kValueBlock;
    const uint32_t ntok = static_cast<uint32_t>(std::min<uint64_t>(kValueBlock, seq - t0));
    // packed key tokens of the block and the key groups they lie in
    const uint32_t nk = t0 < s.kq ? static_cast<uint32_t>(std::min<uint64_t>(kValueBlock, s.kq - t0)) : 0u;
    const uint64_t g_lo = t0 / G;
    if (nk > 0) {
      const uint32_t* kc = c.kcodes + unit * geo.kcodes_unit() + t0 * kw;
      for (uint32_t i = threadIdx.x; i < nk * kw; i += blockDim.x) skw[i] = kc[i];
      const uint32_t ng = static_cast<uint32_t>((t0 + nk - 1) / G - g_lo + 1);
      const float2* kp = reinterpret_cast<const float2*>(c.kparams + unit * geo.kparams_unit()) + g_lo * D;
      for (uint32_t i = threadIdx.x; i < ng * D; i += blockDim.x) skp[i] = kp[i];
    }
    if (t0 < s.vq) {
      const uint32_t* vc = c.vcodes + unit * geo.vcodes_unit() + tb * D * vw;
      for (uint32_t i = threadIdx.x; i < D * vw; i += blockDim.x) svw[(i % vw) * L.vrow + i / vw] = vc[i];
      const float2* vp = reinterpret_cast<const float2*>(c.vparams + unit * geo.vparams_unit()) + tb * ncg * kValueBlock;
      for (uint32_t i = threadIdx.x; i < ncg * kValueBlock; i += blockDim.x) svp[i] = vp[i];
    }
    __syncthreads();
    for (uint32_t r = threadIdx.x; r < ntok * q4; r += blockDim.x) {
      const uint32_t tt = r / q4, d0 = (r % q4) * 4;
      const uint64_t t = t0 + tt;
      float k[4], v[4];
      if (tt < nk) {
        // one code word holds the four channels (ppw >= 4); their (scale, zero) pairs are 32
        // contiguous bytes
        const uint32_t word = skw[tt * kw + d0 / ppw];
        const float4* pp = reinterpret_cast<const float4*>(skp + (t / G - g_lo) * D + d0);
        const float4 p01 = pp[0], p23 = pp[1];
        const float sc[4] = {p01.x, p01.z, p23.x, p23.z}, zr[4] = {p01.y, p01.w, p23.y, p23.w};
#pragma unroll
        for (int e = 0; e < 4; ++e)
          k[e] = fmaf(static_cast<float>((word >> code_shift(bits, (d0 + e) % ppw)) & mask), sc[e], zr[e]);
      } else {
        const float4 x = *reinterpret_cast<const float4*>(c.kres + ((uint64_t)unit * R + (t - s.kq)) * D + d0);
        k[0] = x.x; k[1] = x.y; k[2] = x.z; k[3] = x.w;
      }
      if (t < s.vq) {
        const uint32_t sh = code_shift(bits, tt % ppw);
        const float2 sz = svp[(d0 / G) * kValueBlock + tt];  // one group holds the four (G % 4 == 0)
        const uint4 w = *reinterpret_cast<const uint4*>(svw + (tt / ppw) * L.vrow + d0);
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = fmaf(static_cast<float>((ws[e] >> sh) & mask), sz.x, sz.y);
      } else {
        const float4 x = *reinterpret_cast<const float4*>(
            c.vring + ((uint64_t)unit * R + (s.vhead + (t - s.vq)) % R) * D + d0);
        v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
      }
      const uint64_t o = ((uint64_t)unit * seq + t) * D + d0;
      *reinterpret_cast<float4*>(keys + o) = make_float4(k[0], k[1], k[2], k[3]);
      *reinterpret_cast<float4*>(values + o) = make_float4(v[0], v[1], v[2], v[3]);
    }
    __syncthreads();  // the staging buffer is refilled for the next block
  }
}

// The same, one element per thread, for output arrays not 16-byte aligned.
__global__ void __launch_bounds__(kThreads)
    k_dequant_cache_elem(CacheView c, SeqState s, uint64_t seq, float* keys, float* values) {
  const Geometry& geo = c.geo;
  const uint32_t D = geo.D, G = geo.G, R = geo.R, bits = geo.bits, ppw = geo.ppw();
  const uint32_t kw = geo.kwords_per_token(), vw = geo.vwords_per_channel(), ncg = geo.ncg();
  const uint32_t mask = geo.levels();
  const uint64_t per_unit = seq * D;
  const uint64_t total = per_unit * geo.units;
  for (uint64_t idx = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (uint64_t)gridDim.x * blockDim.x) {
    const uint32_t unit = idx / per_unit;
    const uint64_t r = idx % per_unit;
    const uint64_t t = r / D;
    const uint32_t d = r % D;
    float k, v;
    if (t < s.kq) {
      const uint32_t word = c.kcodes[unit * geo.kcodes_unit() + t * kw + d / ppw];
      const float code = static_cast<float>((word >> code_shift(bits, d % ppw)) & mask);
      const float2 sz = reinterpret_cast<const float2*>(c.kparams + unit * geo.kparams_unit())[(t / G) * D + d];
      k = fmaf(code, sz.x, sz.y);
    } else {
      k = c.kres[((uint64_t)unit * R + (t - s.kq)) * D + d];
    }
    if (t < s.vq) {
      const uint64_t tb = t / kValueBlock;
      const uint32_t tt = t % kValueBlock;
      const uint32_t word = c.vcodes[unit * geo.vcodes_unit() + (tb * D + d) * vw + tt / ppw];
      const float code = static_cast<float>((word >> code_shift(bits, tt % ppw)) & mask);
      const float2 sz = reinterpret_cast<const float2*>(c.vparams + unit * geo.vparams_unit())
          [(tb * ncg + d / G) * kValueBlock + tt];
      v = fmaf(code, sz.x, sz.y);
    } else {
      v = c.vring[((uint64_t)unit * R + (s.vhead + (t - s.vq)) % R) * D + d];
    }
    keys[idx] = k;
    values[idx] = v;
  }
}

// ------------------------------------------------------------------ standalone codec (reference order)
// The wave forms (head_dim = 64*CPL, CPL = 1, 2, 4): a lane holds channels CPL*lane .. +CPL-1
// of each row in registers, as the cache's quantizers do, and the codes are packed straight
// into the reference order. Units are contiguous in both the input and the output, so the
// kernels index groups (keys) and rows (values) over all units at once.

template <int N>
__device__ __forceinline__ void store_words(uint32_t* p, const uint32_t (&w)[N]) {
  typedef uint32_t u4v __attribute__((ext_vector_type(4)));
  typedef uint32_t u2v __attribute__((ext_vector_type(2)));
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int i = 0; i < N; i += 4) *reinterpret_cast<u4v*>(p + i) = u4v{w[i], w[i + 1], w[i + 2], w[i + 3]};
  } else if constexpr (N % 2 == 0) {
#pragma unroll
    for (int i = 0; i < N; i += 2) *reinterpret_cast<u2v*>(p + i) = u2v{w[i], w[i + 1]};
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) p[i] = w[i];
  }
}

// quantize_per_channel (src/quant.rs:153-191 -> append_key_block :275-328): wave per group
// (grid-stride over all units' groups). Word (q*D + d)*ipc + w of group q holds tokens
// w*ppw .. w*ppw+ppw-1 of channel d, first token in the low bits: all of them are the lane's
// own codes, so a lane packs its CPL*ipc consecutive words and stores them in one go.
template <int BITS, int CPL, int GG>
__global__ void __launch_bounds__(kThreads)
    k_codec_keys_wave(const float* data, uint64_t groups, uint32_t* codes, float* params) {
  constexpr uint32_t D = 64 * CPL, PPW = 32 / BITS, IPC = GG / PPW;
  constexpr uint32_t kLevels = (1u << BITS) - 1u;
  constexpr float levels = static_cast<float>(kLevels);
  const uint32_t lane = threadIdx.x % 64;
  for (uint64_t q = (uint64_t)blockIdx.x * 4 + threadIdx.x / 64; q < groups; q += (uint64_t)gridDim.x * 4) {
    const float* rows = data + q * GG * D;
    float x[GG][CPL];
#pragma unroll
    for (int t = 0; t < GG; ++t) load_lane<CPL>(rows + (uint64_t)t * D, lane, x[t]);
    float2* pp = reinterpret_cast<float2*>(params) + q * D + CPL * lane;
    uint32_t w[CPL * IPC];
    float mns[CPL], mxs[CPL];
    bool zero_min = false;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      float mn = INFINITY, mx = -INFINITY;
#pragma unroll
      for (int t = 0; t < GG; ++t) {
        mn = fminf(mn, x[t][j]);
        mx = fmaxf(mx, x[t][j]);
      }
      mns[j] = mn;
      mxs[j] = mx;
      zero_min |= mn == 0.f;
    }
    if (__ballot(zero_min)) {  // rare, and wave-uniform: a zero minimum takes its first zero's sign
#pragma unroll
      for (int j = 0; j < CPL; ++j)
        if (mns[j] == 0.f) mns[j] = first_zero(rows + CPL * lane + j, D, GG);
    }
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const float mn = mns[j];
      const float scale = scale_of(mxs[j] - mn, levels), inv = quant_inv(scale);
      pp[j] = make_float2(scale, mn);
#pragma unroll
      for (int k = 0; k < (int)IPC; ++k) {
        uint32_t word = 0;
#pragma unroll
        for (int i = 0; i < (int)PPW; ++i)
          word |= quant_code_fast(x[k * PPW + i][j], mn, scale, inv, kLevels) << (BITS * i);
        w[j * IPC + k] = word;
      }
    }
    store_words<CPL * IPC>(codes + (q * D + CPL * lane) * IPC, w);
  }
}

// quantize_per_token (src/quant.rs:193-233 -> append_value_block :330-377): wave per 16
// consecutive rows (grid-stride over all units' rows). Group min/max as the cache's value
// quantizer takes them (the 16-lane butterfly when a channel group is a DPP row). Word
// r*(D/ppw) + j of row r holds channels j*ppw .. j*ppw+ppw-1, first channel in the low bits:
// the LPW lanes of a word OR their parts (DPP), lane m keeps rows p = m (mod LPW), and every
// store writes 64 consecutive words; (scale, zero) of (row r, group cg) at r*(D/G) + cg.
template <int BITS, int CPL, int GG>
__global__ void __launch_bounds__(kThreads)
    k_codec_values_wave(const float* data, uint64_t rows, uint32_t* codes, float* params) {
  constexpr uint32_t D = 64 * CPL, PPW = 32 / BITS, NCG = D / GG;
  constexpr uint32_t LPW = PPW / CPL;  // lanes per code word
  constexpr uint32_t KW = D / PPW;     // words per row (= 64 / LPW)
  constexpr uint32_t NS = 16 / LPW;    // words kept per lane
  constexpr uint32_t L = GG / CPL;     // lanes per channel group
  constexpr uint32_t kLevels = (1u << BITS) - 1u;
  constexpr float levels = static_cast<float>(kLevels);
  const uint32_t lane = threadIdx.x % 64;
  const uint32_t cg = CPL * lane / GG;
  const uint32_t m = lane % LPW;
  const uint64_t slabs = (rows + 15) / 16;
  for (uint64_t sl = (uint64_t)blockIdx.x * 4 + threadIdx.x / 64; sl < slabs; sl += (uint64_t)gridDim.x * 4) {
    const uint64_t r0 = sl * 16;
    const uint32_t nvalid = static_cast<uint32_t>(rows - r0 < 16 ? rows - r0 : 16);
    float x[16][CPL];
#pragma unroll
    for (int p = 0; p < 16; ++p) {
      const uint32_t pc = (uint32_t)p < nvalid ? (uint32_t)p : nvalid - 1;  // rows past the end: the last
      load_lane<CPL>(data + (r0 + pc) * D, lane, x[p]);
    }
    uint32_t keep[NS];
#pragma unroll
    for (int k = 0; k < (int)NS; ++k) keep[k] = 0;
    float2* pp = reinterpret_cast<float2*>(params);
    if constexpr (L == 16) {
      float pmn[16], pmx[16];
#pragma unroll
      for (int p = 0; p < 16; ++p) {
        pmn[p] = pmx[p] = x[p][0];
#pragma unroll
        for (int j = 1; j < CPL; ++j) minmax_with(pmn[p], pmx[p], x[p][j], x[p][j]);
      }
      float mn_r, mx_r;
      row_minmax16(pmn, pmx, mn_r, mx_r);
      const uint32_t r = lane % 16;
      if (__ballot(mn_r == 0.f)) {  // rare, and wave-uniform: row r's first zero gives the sign
        if (mn_r == 0.f && r < nvalid) mn_r = first_zero(data + (r0 + r) * D + cg * GG, 1, GG);
      }
      const float scale_r = scale_of(mx_r - mn_r, levels);
      const float inv_r = quant_inv(scale_r);
      if (r < nvalid) pp[(r0 + r) * NCG + cg] = make_float2(scale_r, mn_r);
#pragma unroll
      for (int p = 0; p < 16; ++p) {
        const float scale = row_bcast(scale_r, p), inv = row_bcast(inv_r, p), zero = row_bcast(mn_r, p);
        uint32_t part = 0;
#pragma unroll
        for (int j = 0; j < CPL; ++j)
          part |= quant_code_fast(x[p][j], zero, scale, inv, kLevels) << (BITS * ((CPL * lane + j) % PPW));
        part = group_or<LPW>(part);
        if (m == (uint32_t)p % LPW) keep[p / LPW] = part;
      }
    } else {
#pragma unroll
      for (int p = 0; p < 16; ++p) {
        float mn = x[p][0], mx = x[p][0];
#pragma unroll
        for (int j = 1; j < CPL; ++j) minmax_with(mn, mx, x[p][j], x[p][j]);
        group_minmax<L>(mn, mx);
        if (__ballot(mn == 0.f)) {  // rare, and wave-uniform: row p's first zero gives the sign
          if (mn == 0.f && (uint32_t)p < nvalid) mn = first_zero(data + (r0 + p) * D + cg * GG, 1, GG);
        }
        const float scale = scale_of(mx - mn, levels), inv = quant_inv(scale);
        if (lane % L == 0 && (uint32_t)p < nvalid) pp[(r0 + p) * NCG + cg] = make_float2(scale, mn);
        uint32_t part = 0;
#pragma unroll
        for (int j = 0; j < CPL; ++j)
          part |= quant_code_fast(x[p][j], mn, scale, inv, kLevels) << (BITS * ((CPL * lane + j) % PPW));
        part = group_or<LPW>(part);
        if (m == (uint32_t)p % LPW) keep[p / LPW] = part;
      }
    }
#pragma unroll
    for (int k = 0; k < (int)NS; ++k) {
      const uint32_t p = k * LPW + m;
      if (p < nvalid) codes[(r0 + p) * KW + lane / LPW] = keep[k];
    }
  }
}

// The general forms (any head_dim and group): one workgroup per (unit, group) for keys, one
// thread per (row, channel group) for values.

// quantize_per_channel (src/quant.rs:153-191 -> append_key_block :275-328), one workgroup per
// (unit, group), words (g*D + d)*ipc + w.
__global__ void __launch_bounds__(kThreads)
    k_quant_ref_keys(const float* data, uint64_t tokens, uint32_t D, uint32_t bits, uint32_t G,
                     uint32_t* codes, float* params) {
  extern __shared__ uint8_t codes_lds[];  // [G][D]
  const uint64_t ngroups = tokens / G;
  const uint32_t unit = blockIdx.x / ngroups;
  const uint64_t g = blockIdx.x % ngroups;
  const float levels = static_cast<float>((1u << bits) - 1u);
  const float* rows = data + (unit * tokens + g * G) * D;
  float2* pp = reinterpret_cast<float2*>(params) + (unit * ngroups + g) * D;
  for (uint32_t d = threadIdx.x; d < D; d += blockDim.x) {
    float mn = INFINITY, mx = -INFINITY;
    for (uint32_t t = 0; t < G; ++t) {
      const float x = rows[(uint64_t)t * D + d];
      mn = x < mn ? x : mn;  // keeps the first of equal minima (the first zero)
      mx = fmaxf(mx, x);
    }
    const float scale = scale_of(mx - mn, levels);
    pp[d] = make_float2(scale, mn);
    for (uint32_t t = 0; t < G; ++t)
      codes_lds[t * D + d] = static_cast<uint8_t>(quant_code(rows[(uint64_t)t * D + d], mn, scale, levels));
  }
  __syncthreads();
  const uint32_t ppw = 32 / bits, ipc = G / ppw;
  uint32_t* out = codes + (unit * ngroups + g) * D * ipc;
  for (uint32_t idx = threadIdx.x; idx < D * ipc; idx += blockDim.x) {
    const uint32_t d = idx / ipc, w = idx % ipc;
    uint32_t word = 0;
    for (uint32_t i = 0; i < ppw; ++i)
      word |= static_cast<uint32_t>(codes_lds[(w * ppw + i) * D + d]) << (bits * i);
    out[idx] = word;
  }
}

// quantize_per_token (src/quant.rs:193-233 -> append_value_block :330-377): one thread per
// (unit, token, channel group) owns its ipg words.
__global__ void __launch_bounds__(kThreads)
    k_quant_ref_values(const float* data, uint32_t units, uint64_t tokens, uint32_t D,
                       uint32_t bits, uint32_t G, uint32_t* codes, float* params) {
  const uint32_t ncg = D / G, ppw = 32 / bits, ipg = G / ppw;
  const float levels = static_cast<float>((1u << bits) - 1u);
  const uint64_t total = (uint64_t)units * tokens * ncg;
  for (uint64_t idx = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (uint64_t)gridDim.x * blockDim.x) {
    const float* grp = data + idx * G;  // (unit*tokens + t)*D + cg*G == idx*G
    float mn = INFINITY, mx = -INFINITY;
    for (uint32_t e = 0; e < G; ++e) {
      mn = grp[e] < mn ? grp[e] : mn;  // keeps the first of equal minima (the first zero)
      mx = fmaxf(mx, grp[e]);
    }
    const float scale = scale_of(mx - mn, levels);
    reinterpret_cast<float2*>(params)[idx] = make_float2(scale, mn);
    for (uint32_t w = 0; w < ipg; ++w) {
      uint32_t word = 0;
      for (uint32_t i = 0; i < ppw; ++i)
        word |= quant_code(grp[w * ppw + i], mn, scale, levels) << (bits * i);
      codes[idx * ipg + w] = word;
    }
  }
}

// QuantizedTensor::dequantize (src/quant.rs:124-150 via dequant_keys/values :379-451).
__global__ void __launch_bounds__(kThreads)
    k_dequant_ref(const uint32_t* codes, const float* params, uint32_t units, uint64_t tokens,
                  uint32_t D, uint32_t bits, uint32_t G, int per_channel, float* out) {
  const uint32_t ppw = 32 / bits, mask = (1u << bits) - 1u, ncg = D / G, ipg = G / ppw;
  const uint64_t total = (uint64_t)units * tokens * D;
  for (uint64_t idx = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t ut = idx / D;  // unit*tokens + t
    const uint32_t d = idx % D;
    const uint32_t unit = ut / tokens;
    const uint64_t t = ut % tokens;
    uint32_t word, shift;
    float2 sz;
    if (per_channel) {
      const uint64_t g = t / G;
      const uint32_t tg = t % G;
      const uint64_t base = (unit * (tokens / G) + g) * D + d;  // (g*D + d) within the unit
      word = codes[base * ipg + tg / ppw];
      shift = bits * (tg % ppw);
      sz = reinterpret_cast<const float2*>(params)[base];
    } else {
      const uint64_t gi = ut * ncg + d / G;
      word = codes[gi * ipg + (d % G) / ppw];
      shift = bits * (d % ppw);
      sz = reinterpret_cast<const float2*>(params)[gi];
    }
    out[idx] = fmaf(static_cast<float>((word >> shift) & mask), sz.x, sz.y);
  }
}

// QuantizedTensor::pytorch_codes for keys (src/quant.rs:81-94): out[tp][d] = word (g, d, w)
// with tp = g*ipc + w. Values are already in that order (src/quant.rs:95-109).
__global__ void __launch_bounds__(kThreads)
    k_pytorch_keys(const uint32_t* codes, uint32_t units, uint64_t tokens, uint32_t D, uint32_t bits,
                   uint32_t G, uint32_t* out) {
  const uint32_t ppw = 32 / bits, ipc = G / ppw;
  const uint64_t t_pack = tokens / ppw;
  const uint64_t total = (uint64_t)units * t_pack * D;
  for (uint64_t idx = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t ut = idx / D;
    const uint32_t d = idx % D;
    const uint32_t unit = ut / t_pack;
    const uint64_t tp = ut % t_pack;
    const uint64_t g = tp / ipc;
    const uint32_t w = tp % ipc;
    out[idx] = codes[unit * (t_pack * D) + (g * D + d) * ipc + w];
  }
}

}  // namespace

// ------------------------------------------------------------------ launchers

hipError_t launch_copy_rows(const Geometry& g, RowSource src, float* dst, uint32_t dst_slot,
                            uint32_t count, hipStream_t stream) {
  if (count == 0) return hipSuccess;
  const bool vec = (reinterpret_cast<uintptr_t>(src.base) % 16 == 0) &&
                   (reinterpret_cast<uintptr_t>(dst) % 16 == 0) && (g.D % 4 == 0) &&
                   (src.stride_unit % 4 == 0);
  if (vec) {
    const uint64_t work = (uint64_t)g.units * count * (g.D / 4);
    k_copy_rows<4><<<grid_for(work), kThreads, 0, stream>>>(src, dst, g.R, g.D, g.units, dst_slot, count);
  } else {
    const uint64_t work = (uint64_t)g.units * count * g.D;
    k_copy_rows<1><<<grid_for(work), kThreads, 0, stream>>>(src, dst, g.R, g.D, g.units, dst_slot, count);
  }
  return hipGetLastError();
}

hipError_t launch_decode_append(const CacheView& c, const float* keys, const float* values,
                                uint32_t kslot, uint32_t vslot, bool evict, uint64_t vq,
                                hipStream_t stream) {
  const Geometry& g = c.geo;
  if (g.D % 64 != 0 || g.D > 256 || 64 % g.G != 0) return hipErrorNotSupported;
  k_decode_append<<<g.units, g.D, 0, stream>>>(c, keys, values, kslot, vslot, evict ? 1u : 0u, vq);
  return hipGetLastError();
}

hipError_t launch_raise_row_max(const CacheView& c, uint32_t kres, uint32_t vres, uint32_t vhead,
                                hipStream_t stream) {
  if (kres == 0 && vres == 0) return hipSuccess;
  k_raise_row_max<<<c.geo.units * 2, kThreads, 0, stream>>>(c, kres, vres, vhead);
  return hipGetLastError();
}

bool rows_vec4(const RowSource& r, uint32_t D) {
  return reinterpret_cast<uintptr_t>(r.base) % 16 == 0 && D % 4 == 0 && r.stride_unit % 4 == 0;
}

template <int BITS>
bool keys_wave_bits(uint32_t cpl, uint32_t G, unsigned grid, hipStream_t stream, const CacheView& c,
                    const RowSource& src, uint64_t g0, uint32_t ngroups, uint32_t spans) {
  switch (cpl * 1000 + G) {
    case 1016: k_quant_keys_wave<BITS, 1, 16><<<grid, kThreads, 0, stream>>>(c, src, g0, ngroups, spans); return true;
    case 1032: k_quant_keys_wave<BITS, 1, 32><<<grid, kThreads, 0, stream>>>(c, src, g0, ngroups, spans); return true;
    case 1064: k_quant_keys_wave<BITS, 1, 64><<<grid, kThreads, 0, stream>>>(c, src, g0, ngroups, spans); return true;
    case 2016: k_quant_keys_wave<BITS, 2, 16><<<grid, kThreads, 0, stream>>>(c, src, g0, ngroups, spans); return true;
    case 2032: k_quant_keys_wave<BITS, 2, 32><<<grid, kThreads, 0, stream>>>(c, src, g0, ngroups, spans); return true;
    case 2064: k_quant_keys_wave<BITS, 2, 64><<<grid, kThreads, 0, stream>>>(c, src, g0, ngroups, spans); return true;
    case 4016: k_quant_keys_wave<BITS, 4, 16><<<grid, kThreads, 0, stream>>>(c, src, g0, ngroups, spans); return true;
    case 4032: k_quant_keys_wave<BITS, 4, 32><<<grid, kThreads, 0, stream>>>(c, src, g0, ngroups, spans); return true;
    default: return false;
  }
}

bool keys_wave_dispatch(uint32_t bits, uint32_t cpl, uint32_t G, unsigned grid, hipStream_t stream,
                        const CacheView& c, const RowSource& src, uint64_t g0, uint32_t ngroups,
                        uint32_t spans) {
  switch (bits) {
    case 2: return keys_wave_bits<2>(cpl, G, grid, stream, c, src, g0, ngroups, spans);
    case 4: return keys_wave_bits<4>(cpl, G, grid, stream, c, src, g0, ngroups, spans);
    case 8: return keys_wave_bits<8>(cpl, G, grid, stream, c, src, g0, ngroups, spans);
    default: return false;
  }
}

template <int BITS>
bool values_wave_bits(uint32_t cpl, uint32_t G, unsigned grid, uint32_t spans, hipStream_t stream, const CacheView& c,
                      const RowSource& ring, uint32_t n_ring, const RowSource& in, uint64_t vq0,
                      uint64_t n, uint64_t blk0, uint32_t nblk) {
#define KIVI_VW(C, GG)                                                                              \
  case C * 1000 + GG:                                                                               \
    k_quant_values_wave<BITS, C, GG><<<grid, kThreads, 0, stream>>>(c, ring, n_ring, in, vq0, n,  \
                                                                    blk0, nblk, spans);            \
    return true;
  switch (cpl * 1000 + G) {
    KIVI_VW(1, 16) KIVI_VW(1, 32) KIVI_VW(1, 64)
    KIVI_VW(2, 16) KIVI_VW(2, 32) KIVI_VW(2, 64)
    KIVI_VW(4, 16) KIVI_VW(4, 32)
    default: return false;
  }
#undef KIVI_VW
}

hipError_t launch_quant_keys(const CacheView& c, RowSource src, uint64_t g0, uint32_t ngroups,
                             hipStream_t stream) {
  if (ngroups == 0) return hipSuccess;
  const uint64_t blocks = (uint64_t)c.geo.units * ngroups;
  const size_t codes = ((size_t)c.geo.G * c.geo.D + 15) / 16 * 16;
  const bool staged = (size_t)c.geo.G * (c.geo.D + 1) <= kStageFloats;
  const size_t lds = codes + (staged ? (size_t)c.geo.G * (c.geo.D + 1) * sizeof(float) : 0);
  const double rows = (double)blocks * c.geo.G;
  TimedLaunch timed(KIVI_KERNEL_QUANT_KEYS, stream,
                    rows * c.geo.D * (4.0 + c.geo.bits / 8.0) + (double)blocks * c.geo.D * 8.0);
  const uint32_t cpl = c.geo.D / 64;
  const bool lane_aligned = c.geo.D % 64 == 0 && reinterpret_cast<uintptr_t>(src.base) % (4 * cpl) == 0 &&
                            src.stride_unit % (4 * cpl) == 0 && blocks <= (1ull << 31);
  if (lane_aligned) {
    const uint32_t spans = (ngroups + kKeySpan - 1) / kKeySpan;
    const unsigned grid = c.geo.units * spans;
    if (keys_wave_dispatch(c.geo.bits, cpl, c.geo.G, grid, stream, c, src, g0, ngroups, spans))
      return hipGetLastError();
  }
  k_quant_keys<<<static_cast<unsigned>(blocks), kThreads, lds, stream>>>(c, src, g0, ngroups, staged ? 1u : 0u,
                                                                        rows_vec4(src, c.geo.D) ? 1u : 0u);
  return hipGetLastError();
}

hipError_t launch_quant_values(const CacheView& c, RowSource ring, uint32_t n_ring, RowSource in,
                               uint64_t n_in, uint64_t vq0, hipStream_t stream) {
  const uint64_t n = n_ring + n_in;
  if (n == 0) return hipSuccess;
  const uint64_t blk0 = vq0 / kValueBlock;
  const uint64_t blk1 = (vq0 + n - 1) / kValueBlock;
  const uint32_t nblk = static_cast<uint32_t>(blk1 - blk0 + 1);
  const uint64_t blocks = (uint64_t)c.geo.units * nblk;
  const uint32_t D = c.geo.D;
  const uint32_t TB = std::max<uint32_t>(1, std::min<uint32_t>(kValueBlock, kStageFloats / (D + 1)));
  const size_t lds = ((size_t)kValueBlock * D + 15) / 16 * 16 + (size_t)TB * (D + 1) * sizeof(float);
  const bool vec4 = rows_vec4(ring, D) && (n_in == 0 || rows_vec4(in, D));
  {
    const hipError_t e = raise_lds_limit(reinterpret_cast<const void*>(&k_quant_values), lds);
    if (e != hipSuccess) return e;
  }
  const double rows = (double)c.geo.units * n;
  TimedLaunch timed(KIVI_KERNEL_QUANT_VALUES, stream,
                    rows * (c.geo.D * (4.0 + c.geo.bits / 8.0) + c.geo.ncg() * 8.0));
  const uint32_t cpl = D / 64;
  const uint32_t lanes_per_group = cpl > 0 ? c.geo.G / cpl : 0;
  auto aligned = [&](const RowSource& r) {
    return reinterpret_cast<uintptr_t>(r.base) % (4 * cpl) == 0 && r.stride_unit % (4 * cpl) == 0;
  };
  if (D % 64 == 0 && (cpl == 1 || cpl == 2 || cpl == 4) && c.geo.G % cpl == 0 && lanes_per_group <= 64 &&
      (lanes_per_group & (lanes_per_group - 1)) == 0 && aligned(ring) && (n_in == 0 || aligned(in))) {
    const uint32_t spans = (nblk + kValueSpan - 1) / kValueSpan;
    const unsigned nb = c.geo.units * spans;
    const uint32_t G = c.geo.G;
    bool done = false;
    switch (c.geo.bits) {
      case 2: done = values_wave_bits<2>(cpl, G, nb, spans, stream, c, ring, n_ring, in, vq0, n, blk0, nblk); break;
      case 4: done = values_wave_bits<4>(cpl, G, nb, spans, stream, c, ring, n_ring, in, vq0, n, blk0, nblk); break;
      case 8: done = values_wave_bits<8>(cpl, G, nb, spans, stream, c, ring, n_ring, in, vq0, n, blk0, nblk); break;
      default: break;
    }
    if (done) return hipGetLastError();
  }
  k_quant_values<<<static_cast<unsigned>(blocks), kThreads, lds, stream>>>(c, ring, n_ring, in, vq0, n,
                                                                         blk0, nblk, TB, vec4 ? 1u : 0u);
  return hipGetLastError();
}

hipError_t launch_export_keys(const CacheView& c, uint64_t kq, uint32_t* codes, float* params,
                              hipStream_t stream) {
  const Geometry& g = c.geo;
  if (kq == 0) return hipSuccess;
  if (codes != nullptr) {
    // staged words per group: kw rows of G + 4 tokens, then the n output words when both
    // fit the budget (else the output words go straight to memory)
    const uint32_t np = g.kwords_per_token() * (g.G + 4), n = g.G * g.kwords_per_token();
    const uint32_t stage_out = np + n <= kExportLdsWords ? 1u : 0u;
    const uint32_t per_group = np + (stage_out ? n : 0u);
    const uint32_t per = std::max(1u, std::min(kExportGroups, kExportLdsWords / per_group));
    const uint64_t slices = (kq / g.G + per - 1) / per;
    const size_t lds = (size_t)per * per_group * sizeof(uint32_t);
    const dim3 grid(static_cast<unsigned>(std::min<uint64_t>(slices, 1u << 30)), std::min(g.units, 65535u));
    const void* f = g.bits == 2 ? reinterpret_cast<const void*>(&k_export_keys<2>)
                    : g.bits == 4 ? reinterpret_cast<const void*>(&k_export_keys<4>)
                                  : reinterpret_cast<const void*>(&k_export_keys<8>);
    hipError_t e = raise_lds_limit(f, lds);
    if (e != hipSuccess) return e;
    if (g.bits == 2) k_export_keys<2><<<grid, kThreads, lds, stream>>>(c, kq, per, stage_out, codes);
    else if (g.bits == 4) k_export_keys<4><<<grid, kThreads, lds, stream>>>(c, kq, per, stage_out, codes);
    else k_export_keys<8><<<grid, kThreads, lds, stream>>>(c, kq, per, stage_out, codes);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (params != nullptr) {
    const size_t bytes = (kq / g.G) * g.D * 2 * sizeof(float);
    return copy_units(params, bytes, c.kparams, g.kparams_unit() * sizeof(float), bytes, g.units, stream);
  }
  return hipSuccess;
}

hipError_t launch_export_values(const CacheView& c, uint64_t vq, uint32_t* codes, float* params,
                                hipStream_t stream) {
  const Geometry& g = c.geo;
  if (vq == 0) return hipSuccess;
  // Codes and params come out of one pass; a null codes array still needs the pass.
  uint32_t* tmp = nullptr;
  if (codes == nullptr) {
    if (params == nullptr) return hipSuccess;
    hipError_t e = hipMallocAsync(reinterpret_cast<void**>(&tmp), g.units * vq * (g.D / g.ppw()) * 4, stream);
    if (e != hipSuccess) return e;
    codes = tmp;
  }
  const uint64_t nblk = (vq + kValueBlock - 1) / kValueBlock;
  // staged words per block: VW rows of D + 4 channels (a block of the widest heads, D = 1024
  // at 8 bits, stages 16448 words: 64.3 KB), then the output words when both fit the budget
  const uint32_t vw = g.vwords_per_channel();
  const uint32_t np = vw * (g.D + 4), n = g.D * vw;
  const uint32_t stage_out = np + n <= kExportLdsWords ? 1u : 0u;
  const uint32_t per_block = np + (stage_out ? n : 0u);
  const uint32_t per = std::max(1u, std::min(kExportBlocks, kExportLdsWords / per_block));
  const uint64_t slices = (nblk + per - 1) / per;
  const size_t lds = (size_t)per * per_block * sizeof(uint32_t);
  const dim3 grid(static_cast<unsigned>(std::min<uint64_t>(slices, 1u << 30)), std::min(g.units, 65535u));
  const void* f = g.bits == 2 ? reinterpret_cast<const void*>(&k_export_values<2>)
                  : g.bits == 4 ? reinterpret_cast<const void*>(&k_export_values<4>)
                                : reinterpret_cast<const void*>(&k_export_values<8>);
  hipError_t e = raise_lds_limit(f, lds);
  if (e == hipSuccess) {
    if (g.bits == 2) k_export_values<2><<<grid, kThreads, lds, stream>>>(c, vq, per, stage_out, codes, params);
    else if (g.bits == 4) k_export_values<4><<<grid, kThreads, lds, stream>>>(c, vq, per, stage_out, codes, params);
    else k_export_values<8><<<grid, kThreads, lds, stream>>>(c, vq, per, stage_out, codes, params);
  }
  if (e == hipSuccess) e = hipGetLastError();
  if (tmp != nullptr) {
    hipError_t f = hipFreeAsync(tmp, stream);
    if (e == hipSuccess) e = f;
  }
  return e;
}

hipError_t launch_dequant_cache(const CacheView& c, const SeqState& s, float* keys, float* values,
                                hipStream_t stream) {
  const uint64_t seq = s.kq + s.kres;
  const uint64_t work = seq * (c.geo.D / 4);
  if (work == 0) return hipSuccess;
  const size_t lds = (size_t)dequant_lds(c.geo).total * sizeof(uint32_t);
  // staging beyond the default 64 KB of LDS (wide heads) is asked for, up to 128 KB
  const bool fits = lds <= 131072 && raise_lds_limit(reinterpret_cast<const void*>(&k_dequant_cache), lds) == hipSuccess;
  // unaligned outputs, and blocks whose staging would not fit: one element per thread
  if (reinterpret_cast<uintptr_t>(keys) % 16 != 0 || reinterpret_cast<uintptr_t>(values) % 16 != 0 || !fits) {
    k_dequant_cache_elem<<<grid_for(work * 4 * c.geo.units), kThreads, 0, stream>>>(c, s, seq, keys, values);
    return hipGetLastError();
  }
  const uint64_t blocks = (seq + kValueBlock - 1) / kValueBlock * c.geo.units;
  k_dequant_cache<<<static_cast<unsigned>(std::min<uint64_t>(blocks, 32768)), kThreads, lds, stream>>>(
      c, s, seq, keys, values);
  return hipGetLastError();
}

hipError_t raise_lds_limit(const void* kernel, size_t bytes) {
  if (bytes <= 65536) return hipSuccess;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  static std::mutex mu;
  static std::map<std::pair<const void*, int>, size_t> raised;
  std::lock_guard<std::mutex> lock(mu);
  size_t& have = raised[{kernel, dev}];
  if (have >= bytes) return hipSuccess;
  e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
  if (e == hipSuccess) have = bytes;
  return e;
}

hipError_t copy_units(void* dst, size_t dst_pitch, const void* src, size_t src_pitch, size_t bytes,
                      uint32_t units, hipStream_t stream) {
  if (bytes == 0 || units == 0) return hipSuccess;
  return hipMemcpy2DAsync(dst, dst_pitch, src, src_pitch, bytes, units, hipMemcpyDeviceToDevice,
                          stream);
}

// Wave-form instantiations of the standalone codec: channels per lane 1, 2, 4 and the groups
// the cache's quantizers take (false: the general kernel runs).
#define KIVI_CODEC_CASES(X) X(1, 16) X(1, 32) X(1, 64) X(2, 16) X(2, 32) X(2, 64) X(4, 16) X(4, 32)
template <int BITS>
bool codec_keys_bits(uint32_t cpl, uint32_t G, unsigned grid, hipStream_t stream, const float* data,
                     uint64_t groups, uint32_t* codes, float* params) {
#define KIVI_CK(C, GG)                                                                     \
  case C * 1000 + GG:                                                                      \
    k_codec_keys_wave<BITS, C, GG><<<grid, kThreads, 0, stream>>>(data, groups, codes, params); \
    return true;
  switch (cpl * 1000 + G) {
    KIVI_CODEC_CASES(KIVI_CK)
    default: return false;
  }
#undef KIVI_CK
}
template <int BITS>
bool codec_values_bits(uint32_t cpl, uint32_t G, unsigned grid, hipStream_t stream, const float* data,
                       uint64_t rows, uint32_t* codes, float* params) {
#define KIVI_CV(C, GG)                                                                        \
  case C * 1000 + GG:                                                                         \
    k_codec_values_wave<BITS, C, GG><<<grid, kThreads, 0, stream>>>(data, rows, codes, params); \
    return true;
  switch (cpl * 1000 + G) {
    KIVI_CODEC_CASES(KIVI_CV)
    default: return false;
  }
#undef KIVI_CV
}
#undef KIVI_CODEC_CASES

// Channels per lane of the wave forms for head_dim D (0: none) given the input's alignment.
uint32_t codec_cpl(const float* data, uint32_t D) {
  const uint32_t cpl = D / 64;
  if (D % 64 != 0 || !(cpl == 1 || cpl == 2 || cpl == 4)) return 0;
  return reinterpret_cast<uintptr_t>(data) % (4 * cpl) == 0 ? cpl : 0;
}

hipError_t launch_quant_ref_keys(const float* data, uint32_t units, uint64_t tokens, uint32_t D,
                                 uint32_t bits, uint32_t G, uint32_t* codes, float* params,
                                 hipStream_t stream) {
  const uint64_t blocks = (uint64_t)units * (tokens / G);
  if (blocks == 0) return hipSuccess;
  const double elems = (double)units * tokens * D;
  TimedLaunch timed(KIVI_KERNEL_CODEC_KEYS, stream, elems * (4.0 + bits / 8.0) + (double)blocks * D * 8.0);
  const uint32_t cpl = codec_cpl(data, D);
  if (cpl != 0) {
    const unsigned grid = static_cast<unsigned>(std::min<uint64_t>((blocks + 3) / 4, 1u << 20));
    bool done = false;
    switch (bits) {
      case 2: done = codec_keys_bits<2>(cpl, G, grid, stream, data, blocks, codes, params); break;
      case 4: done = codec_keys_bits<4>(cpl, G, grid, stream, data, blocks, codes, params); break;
      case 8: done = codec_keys_bits<8>(cpl, G, grid, stream, data, blocks, codes, params); break;
      default: break;
    }
    if (done) return hipGetLastError();
  }
  k_quant_ref_keys<<<static_cast<unsigned>(blocks), kThreads, (size_t)G * D, stream>>>(
      data, tokens, D, bits, G, codes, params);
  return hipGetLastError();
}

hipError_t launch_quant_ref_values(const float* data, uint32_t units, uint64_t tokens, uint32_t D,
                                   uint32_t bits, uint32_t G, uint32_t* codes, float* params,
                                   hipStream_t stream) {
  const uint64_t work = (uint64_t)units * tokens * (D / G);
  if (work == 0) return hipSuccess;
  const uint64_t rows = (uint64_t)units * tokens;
  TimedLaunch timed(KIVI_KERNEL_CODEC_VALUES, stream,
                    (double)rows * (D * (4.0 + bits / 8.0) + (double)(D / G) * 8.0));
  const uint32_t cpl = codec_cpl(data, D);
  if (cpl != 0 && G % cpl == 0) {
    const unsigned grid = static_cast<unsigned>(std::min<uint64_t>(((rows + 15) / 16 + 3) / 4, 1u << 20));
    bool done = false;
    switch (bits) {
      case 2: done = codec_values_bits<2>(cpl, G, grid, stream, data, rows, codes, params); break;
      case 4: done = codec_values_bits<4>(cpl, G, grid, stream, data, rows, codes, params); break;
      case 8: done = codec_values_bits<8>(cpl, G, grid, stream, data, rows, codes, params); break;
      default: break;
    }
    if (done) return hipGetLastError();
  }
  k_quant_ref_values<<<grid_for(work), kThreads, 0, stream>>>(data, units, tokens, D, bits, G, codes, params);
  return hipGetLastError();
}

hipError_t launch_dequant_ref(const uint32_t* codes, const float* params, uint32_t units,
                              uint64_t tokens, uint32_t D, uint32_t bits, uint32_t G,
                              int per_channel, float* out, hipStream_t stream) {
  const uint64_t work = (uint64_t)units * tokens * D;
  if (work == 0) return hipSuccess;
  k_dequant_ref<<<grid_for(work), kThreads, 0, stream>>>(codes, params, units, tokens, D, bits, G,
                                                        per_channel, out);
  return hipGetLastError();
}

hipError_t launch_pytorch_order(const uint32_t* codes, uint32_t units, uint64_t tokens, uint32_t D,
                                uint32_t bits, uint32_t G, int per_channel, uint32_t* out,
                                hipStream_t stream) {
  const uint64_t words = (uint64_t)units * tokens * D / (32 / bits);
  if (words == 0) return hipSuccess;
  if (!per_channel)
    return hipMemcpyAsync(out, codes, words * 4, hipMemcpyDeviceToDevice, stream);
  k_pytorch_keys<<<grid_for(words), kThreads, 0, stream>>>(codes, units, tokens, D, bits, G, out);
  return hipGetLastError();
}

}  // namespace kivi
