// kernels_attn.hip — split-K fused decode attention over the packed KIVI cache.
//
// Semantics: KiviCache::attention / RagSession::attention (reference src/cache.rs:224-279,
// src/prefix.rs:228-289, src/attention.rs:47-105). Token order is global: keys
// [0,kq) packed | [kq,seq) fp32 residual | [seq,seq+L) suffix; values [0,vq) packed |
// [vq,seq) fp32 window | suffix. The softmax is computed per split with its own max
// (flash-decoding) and merged exactly by log-sum-exp in a second kernel, so results match
// the reference's two-pass softmax within f32 rounding, never bitwise.
//
// The generic kernel below covers every (bits, G, D, GQA) the reference accepts: each
// thread computes one token's logits in the reference's operation order
// (recon = fma(code, scale, zero); logit = fma(recon, q, logit), channels ascending,
// src/attention.rs:143-177, 289-300), one workgroup per (unit, split).
#include "common.hpp"

#include <algorithm>

namespace kivi {
namespace {

constexpr int kThreads = 256;
constexpr int kHeadsPerPass = 4;

struct AttnArgs {
  CacheView c;
  SeqState st;
  uint64_t seq;
  uint64_t total;       // seq + L
  const float* suffix_k;
  const float* suffix_v;
  uint64_t L;
  uint64_t suffix_stride;  // floats between units of the suffix arrays
  const float* query;   // [batch][QH][D]
  uint32_t qh, heads, gq;
  float scale;
  uint32_t S;           // tokens per split
  uint32_t nsplit;
  float* ws;            // [units][nsplit][gq][D+2]
};

__device__ __forceinline__ float key_at(const AttnArgs& a, uint32_t unit, uint64_t t, uint32_t d) {
  const Geometry& g = a.c.geo;
  if (t < a.st.kq) {
    const uint32_t ppw = g.ppw();
    const uint32_t word = a.c.kcodes[unit * g.kcodes_unit() + t * g.kwords_per_token() + d / ppw];
    const float code = static_cast<float>((word >> (g.bits * (d % ppw))) & g.levels());
    const float2 sz = reinterpret_cast<const float2*>(a.c.kparams + unit * g.kparams_unit())[(t / g.G) * g.D + d];
    return fmaf(code, sz.x, sz.y);
  }
  if (t < a.seq) return a.c.kres[((uint64_t)unit * g.R + (t - a.st.kq)) * g.D + d];
  return a.suffix_k[unit * a.suffix_stride + (t - a.seq) * g.D + d];
}

__device__ __forceinline__ float value_at(const AttnArgs& a, uint32_t unit, uint64_t t, uint32_t d) {
  const Geometry& g = a.c.geo;
  if (t < a.st.vq) {
    const uint32_t ppw = g.ppw();
    const uint64_t tb = t / kValueBlock;
    const uint32_t tt = t % kValueBlock;
    const uint32_t word = a.c.vcodes[unit * g.vcodes_unit() + (tb * g.D + d) * g.vwords_per_channel() + tt / ppw];
    const float code = static_cast<float>((word >> (g.bits * (tt % ppw))) & g.levels());
    const float2 sz = reinterpret_cast<const float2*>(a.c.vparams + unit * g.vparams_unit())
        [(tb * g.ncg() + d / g.G) * kValueBlock + tt];
    return fmaf(code, sz.x, sz.y);
  }
  if (t < a.seq)
    return a.c.vring[((uint64_t)unit * g.R + (a.st.vhead + (t - a.st.vq)) % g.R) * g.D + d];
  return a.suffix_v[unit * a.suffix_stride + (t - a.seq) * g.D + d];
}

__device__ __forceinline__ float warp_max(float v) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ float warp_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// One workgroup per (unit, split). LDS: q [gq][D], logits/weights [gq][S].
__global__ void __launch_bounds__(kThreads) k_attn_generic(AttnArgs a) {
  extern __shared__ float lds[];
  const Geometry& g = a.c.geo;
  const uint32_t D = g.D, gq = a.gq, S = a.S;
  const uint32_t unit = blockIdx.x / a.nsplit;
  const uint32_t split = blockIdx.x % a.nsplit;
  const uint32_t b = unit / a.heads, kvh = unit % a.heads;
  float* q_lds = lds;               // [gq][D]
  float* w_lds = lds + gq * D;      // [gq][S]
  const uint64_t t0 = (uint64_t)split * S;
  const uint32_t ntok = static_cast<uint32_t>(std::min<uint64_t>(S, a.total - t0));

  for (uint32_t i = threadIdx.x; i < gq * D; i += blockDim.x) {
    const uint32_t h = i / D, d = i % D;
    q_lds[i] = a.query[((uint64_t)b * a.qh + kvh * gq + h) * D + d];
  }
  __syncthreads();

  // Logits: one token per thread, heads in passes of kHeadsPerPass.
  const uint32_t passes = (gq + kHeadsPerPass - 1) / kHeadsPerPass;
  for (uint32_t idx = threadIdx.x; idx < ntok * passes; idx += blockDim.x) {
    const uint32_t k = idx % ntok, pass = idx / ntok;
    const uint64_t t = t0 + k;
    const uint32_t h0 = pass * kHeadsPerPass;
    const uint32_t nh = std::min<uint32_t>(kHeadsPerPass, gq - h0);
    float acc[kHeadsPerPass] = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t d = 0; d < D; ++d) {
      const float kv = key_at(a, unit, t, d);
#pragma unroll
      for (int h = 0; h < kHeadsPerPass; ++h)
        if (h < (int)nh) acc[h] = fmaf(kv, q_lds[(h0 + h) * D + d], acc[h]);
    }
#pragma unroll
    for (int h = 0; h < kHeadsPerPass; ++h)
      if (h < (int)nh) w_lds[(h0 + h) * S + k] = acc[h] * a.scale;
  }
  __syncthreads();

  // Per-head max and exp-sum over the split (one wavefront per head).
  const uint32_t lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  float* part = a.ws + ((uint64_t)unit * a.nsplit + split) * gq * (D + 2);
  for (uint32_t h = wave; h < gq; h += blockDim.x / 64) {
    float m = -INFINITY;
    for (uint32_t k = lane; k < ntok; k += 64) m = fmaxf(m, w_lds[h * S + k]);
    m = warp_max(m);
    float l = 0.f;
    for (uint32_t k = lane; k < ntok; k += 64) {
      const float w = expf(w_lds[h * S + k] - m);
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

  // Value mix: one (channel, head pass) per thread, tokens ascending.
  for (uint32_t idx = threadIdx.x; idx < D * passes; idx += blockDim.x) {
    const uint32_t d = idx % D, pass = idx / D;
    const uint32_t h0 = pass * kHeadsPerPass;
    const uint32_t nh = std::min<uint32_t>(kHeadsPerPass, gq - h0);
    float acc[kHeadsPerPass] = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t k = 0; k < ntok; ++k) {
      const float v = value_at(a, unit, t0 + k, d);
#pragma unroll
      for (int h = 0; h < kHeadsPerPass; ++h)
        if (h < (int)nh) acc[h] = fmaf(v, w_lds[(h0 + h) * S + k], acc[h]);
    }
#pragma unroll
    for (int h = 0; h < kHeadsPerPass; ++h)
      if (h < (int)nh) part[(h0 + h) * (D + 2) + d] = acc[h];
  }
}

// Log-sum-exp merge of the split partials: one workgroup per (unit, head).
__global__ void __launch_bounds__(kThreads)
    k_attn_merge(const float* ws, uint32_t nsplit, uint32_t gq, uint32_t D, uint32_t heads,
                 uint32_t qh, float* out) {
  const uint32_t unit = blockIdx.x / gq, h = blockIdx.x % gq;
  const uint32_t b = unit / heads, kvh = unit % heads;
  const float* base = ws + (uint64_t)unit * nsplit * gq * (D + 2) + h * (D + 2);
  const uint64_t stride = (uint64_t)gq * (D + 2);
  float M = -INFINITY;
  for (uint32_t s = 0; s < nsplit; ++s) M = fmaxf(M, base[s * stride + D]);
  float L = 0.f;
  for (uint32_t s = 0; s < nsplit; ++s) L += base[s * stride + D + 1] * expf(base[s * stride + D] - M);
  const float inv = 1.0f / L;
  float* o = out + ((uint64_t)b * qh + kvh * gq + h) * D;
  for (uint32_t d = threadIdx.x; d < D; d += blockDim.x) {
    float acc = 0.f;
    for (uint32_t s = 0; s < nsplit; ++s) acc += base[s * stride + d] * expf(base[s * stride + D] - M);
    o[d] = acc * inv;
  }
}

uint32_t split_tokens(uint32_t gq) {
  uint32_t s = 256;
  while (s > 32 && (uint64_t)gq * s > 8192) s >>= 1;
  return s;
}

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
  a.scale = p.scale;
  a.S = split_tokens(a.gq);
  a.nsplit = static_cast<uint32_t>((a.total + a.S - 1) / a.S);
  a.ws = ws;
  return a;
}

}  // namespace

size_t attention_workspace_floats(const AttnProblem& p) {
  const AttnArgs a = make_args(p, nullptr);
  return (size_t)p.cache.geo.units * a.nsplit * a.gq * (p.cache.geo.D + 2);
}

hipError_t launch_attention(const AttnProblem& p, float* workspace, hipStream_t stream) {
  const AttnArgs a = make_args(p, workspace);
  if (a.total == 0) return hipSuccess;
  const uint32_t units = p.cache.geo.units;
  const size_t lds = ((size_t)a.gq * p.cache.geo.D + (size_t)a.gq * a.S) * sizeof(float);
  k_attn_generic<<<units * a.nsplit, kThreads, lds, stream>>>(a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  k_attn_merge<<<units * a.gq, kThreads, 0, stream>>>(workspace, a.nsplit, a.gq, p.cache.geo.D,
                                                     p.heads, p.qh, p.out);
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
