// common.hpp — device layout of the KIVI cache in HBM and the launch interface shared by
// the HIP kernels (kernels_*.hip) and the host state machine (host.cpp).
//
// Per (batch, kv_head) "unit" the cache holds four packed arrays, each with a fixed
// per-unit capacity of `cap` tokens (cap is a multiple of lcm(64, G)):
//
//   key codes    u32 [cap][D/ppw]           token-major: word (t, j) holds channels
//                                           j*ppw .. j*ppw+ppw-1 of token t, channel
//                                           j*ppw+i at bit code_shift(b, i)
//   key params   f32 [cap/G][D][2]          (scale, zero) per (group, channel) — the
//                                           reference PackedStream order (src/quant.rs:307-311)
//   value codes  u32 [cap/64][D][64/ppw]    channel-major in 64-token blocks: word (blk, d, w)
//                                           holds tokens blk*64 + w*ppw + i of channel d,
//                                           token w*ppw+i at bit code_shift(b, i)
//   value params f32 [cap/64][D/G][64][2]   (scale, zero) per (token, channel group)
//
// with ppw = 32/bits codes per word. Element i of a word sits at bit code_shift(bits, i):
// 4-bit and 8-bit words are byte-sliced (element i in byte i % 4, at bit offset
// bits*(i/4) of that byte), 2-bit words nibble-sliced (element i in nibble i % 8, at bit
// offset 2*(i/8) of that nibble). One shift-and-mask then leaves four (4-bit) or eight
// (2-bit) consecutive elements one per byte or nibble, which the attention kernels convert
// into MFMA operands with the packed fp8 / fp4 converters and no further shuffling.
// Per unit, smax holds the largest key and value scale and the largest key and value
// magnitude quantized so far, in kMaxSlots records (see CacheView and unit_max).
//
// fp32 state per unit: key residual [R][D] (linear, token kq+i in slot i) and the value
// window [R][D] as a ring (token vq+i in slot (vhead+i) % R), so a decode step evicts one
// token without the reference's O(R*D) memmove (src/cache.rs:559-578).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace kivi {

constexpr uint32_t kValueBlock = 64;  // tokens per value code block

// Bit offset of element i (0 <= i < 32/bits) inside a native code word.
__host__ __device__ inline uint32_t code_shift(uint32_t bits, uint32_t i) {
  return bits == 2 ? 4u * (i & 7u) + 2u * (i >> 3) : 8u * (i & 3u) + bits * (i >> 2);
}

// Sign of a zero group minimum. The reference takes minima with f32::min in element order
// (src/quant.rs:303 over a group's tokens, :356 over its channels), which on x86-64 is minss
// with the running minimum as the operand passed through on ties: a group whose minimum is
// zero keeps the sign of its FIRST zero (+0 and -0 compare equal, so a later zero never
// replaces an earlier one). Its stored `zero` carries that sign. The quantize kernels find
// the minimum's value with reductions in any order, and when it is zero (rare) fix its sign
// with one of these. first_zero scans n elements `stride` apart in element order.
__host__ __device__ inline float first_zero(const float* p, uint64_t stride, uint32_t n) {
  for (uint32_t i = 0; i < n; ++i) {
    const float x = p[i * stride];
    if (x == 0.f) return x;
  }
  return 0.f;
}
// One element per lane, aligned groups of L lanes in element order (L a power of two <= 64;
// every lane of the wave active): the group's first zero (0.f when it has none).
__device__ inline float lane_group_first_zero(float x, uint32_t L) {
  const uint32_t lane = __lane_id();
  const uint32_t base = lane & ~(L - 1u);
  const uint64_t zeros = __ballot(x == 0.f);
  const uint64_t mine = L == 64 ? zeros : (zeros >> base) & ((1ull << L) - 1ull);
  const float z = __shfl(x, static_cast<int>(base + (mine ? __ffsll(static_cast<long long>(mine)) - 1 : 0)));
  return mine ? z : 0.f;
}

struct Geometry {
  uint32_t bits;  // 2, 4, 8
  uint32_t G;     // group size
  uint32_t R;     // residual length
  uint32_t D;     // head dim
  uint32_t units; // batch * kv_heads
  uint64_t cap;   // token capacity per unit

  __host__ __device__ uint32_t ppw() const { return 32u / bits; }
  __host__ __device__ uint32_t kwords_per_token() const { return D / ppw(); }
  __host__ __device__ uint32_t vwords_per_channel() const { return kValueBlock / ppw(); }
  __host__ __device__ uint32_t ncg() const { return D / G; }
  __host__ __device__ uint32_t levels() const { return (1u << bits) - 1u; }
  // per-unit element counts
  __host__ __device__ uint64_t kcodes_unit() const { return cap * kwords_per_token(); }
  __host__ __device__ uint64_t kparams_unit() const { return (cap / G) * D * 2; }
  __host__ __device__ uint64_t vcodes_unit() const { return (cap / kValueBlock) * D * vwords_per_channel(); }
  __host__ __device__ uint64_t vparams_unit() const { return cap * ncg() * 2; }
  __host__ __device__ uint64_t residual_unit() const { return (uint64_t)R * D; }
};

// Device pointers of one cache (or a frozen prefix copy).
struct CacheView {
  Geometry geo;
  uint32_t* kcodes;
  float* kparams;
  uint32_t* vcodes;
  float* vparams;
  float* kres;   // [units][R][D]
  float* vring;  // [units][R][D]
  // [kMaxSlots][units][4]: running maxima of the key scales, the value scales, the
  // key |x| and the value |x| ever quantized into each unit (words kMaxKeyScale ..
  // kMaxValueAbs of a slot record; f32 bit patterns of values >= 0, so unsigned order is float
  // order). A writer raises the record its workgroup index selects (max_slot), a reader takes
  // the maximum over the records (unit_max). The attention kernels derive power-of-two operand
  // ranges from them; |x| bounds every dequantized element (up to rounding).
  uint32_t* smax;
};

// The maxima records: record s of every unit in region s ([kMaxSlots][units][4] words), so the
// atomics of one launch spread over kMaxSlots regions: with one record per unit, the records of
// eight units shared one 128-byte line and every quantize workgroup's atomics queued on it
// (batch 1 x 8 heads). A reader takes the maximum over a unit's kMaxSlots records.
constexpr uint32_t kMaxSlots = 8;
constexpr uint32_t kMaxRecordWords = 4;  // key scale, value scale, key |x|, value |x|
constexpr uint32_t kMaxUnitWords = kMaxSlots * kMaxRecordWords;
constexpr uint32_t kMaxKeyScale = 0, kMaxValueScale = 1, kMaxKeyAbs = 2, kMaxValueAbs = 3;

// Record `slot` (mod kMaxSlots) of a unit's maxima.
__device__ __forceinline__ uint32_t* max_slot(const CacheView& c, uint32_t unit, uint32_t slot) {
  return c.smax + ((uint64_t)(slot % kMaxSlots) * c.geo.units + unit) * kMaxRecordWords;
}

// The largest key and value scale of a unit over its records (one pair of words per record,
// both taken at once: the attention kernels need the value scale only after the logits, and a
// second round of loads there would stand on a decode launch's critical path).
__device__ __forceinline__ void unit_scale_max(const CacheView& c, uint32_t unit, float& kmax, float& vmax) {
  const uint32_t* p = c.smax + (uint64_t)unit * kMaxRecordWords;
  const uint64_t stride = (uint64_t)c.geo.units * kMaxRecordWords;
  uint32_t km = 0, vm = 0;
#pragma unroll
  for (uint32_t s = 0; s < kMaxSlots; ++s) {
    const uint2 w = *reinterpret_cast<const uint2*>(p + s * stride);
    km = km > w.x ? km : w.x;
    vm = vm > w.y ? vm : w.y;
  }
  kmax = __uint_as_float(km);
  vmax = __uint_as_float(vm);
}

// Maximum `which` (kMaxKeyScale .. kMaxValueAbs) of a unit over its records.
__device__ __forceinline__ float unit_max(const CacheView& c, uint32_t unit, uint32_t which) {
  const uint32_t* p = c.smax + (uint64_t)unit * kMaxRecordWords + which;
  const uint64_t stride = (uint64_t)c.geo.units * kMaxRecordWords;
  uint32_t m = p[0];
#pragma unroll
  for (uint32_t s = 1; s < kMaxSlots; ++s) m = m > p[s * stride] ? m : p[s * stride];
  return __uint_as_float(m);
}

// Sequence state of a cache at one instant.
struct SeqState {
  uint64_t kq;       // packed key tokens
  uint64_t vq;       // packed value tokens
  uint32_t kres;     // key residual length
  uint32_t vres;     // value window length
  uint32_t vhead;    // ring slot of token vq
};

// Where the fp32 rows of a token range come from: [units][seq][D] starting at `offset`
// (stride_unit = seq*D), or the value ring when ring != 0.
struct RowSource {
  const float* base;
  uint64_t stride_unit;  // floats between units
  uint64_t offset;       // first token
  uint32_t ring;         // 1: slot = (offset + i) % R
};

// ---------------------------------------------------------------- launch timing (timing.cpp)
// Brackets the launches made during its lifetime with HIP events on `stream` when timing
// is enabled (kivi_timing_enable); `family` is a kivi_kernel_family, `bytes` the
// algorithmic bytes of the launch.
class TimedLaunch {
 public:
  TimedLaunch(int family, hipStream_t stream, double bytes);
  ~TimedLaunch();
  TimedLaunch(const TimedLaunch&) = delete;
  TimedLaunch& operator=(const TimedLaunch&) = delete;

 private:
  int family_;
  hipStream_t stream_;
  double bytes_;
  int device_ = 0;
  hipEvent_t start_ = nullptr, end_ = nullptr;
};

// ---------------------------------------------------------------- launches (kernels_quant.hip)
// All return hipSuccess or the launch error; all enqueue on `stream`.

// Copy `count` rows of each unit from src into dst[unit][R][D] slots (dst_slot + i) % R.
hipError_t launch_copy_rows(const Geometry& g, RowSource src, float* dst, uint32_t dst_slot,
                            uint32_t count, hipStream_t stream);

// Quantize `ngroups` key groups per unit from src rows into the native key arrays,
// writing groups g0 .. g0+ngroups-1 (src/quant.rs:275-328 per group).
hipError_t launch_quant_keys(const CacheView& c, RowSource src, uint64_t g0, uint32_t ngroups,
                             hipStream_t stream);

// Quantize `n_ring` ring tokens then `n_in` input tokens per unit as stream tokens
// vq0 .. vq0+n-1 (src/quant.rs:330-377 per token).
hipError_t launch_quant_values(const CacheView& c, RowSource ring, uint32_t n_ring, RowSource in,
                               uint64_t n_in, uint64_t vq0, hipStream_t stream);

// One decode token per unit in one launch (KiviCache::append with one token,
// src/cache.rs:382-484, without a key flush): key row -> residual slot `kslot`; when `evict`,
// the window row in slot `vslot` (stream token `vq`) is quantized into the packed values
// first; the value row then goes to slot `vslot`. keys/values are [units][D]. Needs
// D % 64 == 0, D <= 256 and G dividing 64 (returns hipErrorNotSupported otherwise).
hipError_t launch_decode_append(const CacheView& c, const float* keys, const float* values,
                                uint32_t kslot, uint32_t vslot, bool evict, uint64_t vq,
                                hipStream_t stream);

// Raise each unit's |x| maxima (smax [2] keys, [3] values) over its fp32 rows: key residual
// slots [0, kres), value window slots vhead .. vhead+vres-1 (mod R). A shared prefix does
// this once, so its maxima bound every element its attention dequantizes.
hipError_t launch_raise_row_max(const CacheView& c, uint32_t kres, uint32_t vres, uint32_t vhead,
                                hipStream_t stream);

// Re-pack native streams into the reference PackedStream order, [units][...] concatenated.
hipError_t launch_export_keys(const CacheView& c, uint64_t kq, uint32_t* codes, float* params,
                              hipStream_t stream);
hipError_t launch_export_values(const CacheView& c, uint64_t vq, uint32_t* codes, float* params,
                                hipStream_t stream);

// Dense [units][seq][D] reconstruction (src/cache.rs:282-325).
hipError_t launch_dequant_cache(const CacheView& c, const SeqState& s, float* keys, float* values,
                                hipStream_t stream);

// Let `kernel` launch with `bytes` of dynamic LDS on the current device. The limit is an
// attribute of the kernel on each device (64 KB unless raised); each (kernel, device) pair is
// raised once to the largest size asked for so far, from any thread.
hipError_t raise_lds_limit(const void* kernel, size_t bytes);

// Copy `units` blocks of `bytes` from src (pitch src_pitch) to dst (pitch dst_pitch).
hipError_t copy_units(void* dst, size_t dst_pitch, const void* src, size_t src_pitch, size_t bytes,
                      uint32_t units, hipStream_t stream);

// ---------------------------------------------------------------- standalone codec
// Reference-order streams for quantize_per_channel / quantize_per_token
// (src/quant.rs:153-233): codes/params concatenated over units.
hipError_t launch_quant_ref_keys(const float* data, uint32_t units, uint64_t tokens, uint32_t D,
                                 uint32_t bits, uint32_t G, uint32_t* codes, float* params,
                                 hipStream_t stream);
hipError_t launch_quant_ref_values(const float* data, uint32_t units, uint64_t tokens, uint32_t D,
                                   uint32_t bits, uint32_t G, uint32_t* codes, float* params,
                                   hipStream_t stream);
// QuantizedTensor::dequantize and ::pytorch_codes (src/quant.rs:77-150).
hipError_t launch_dequant_ref(const uint32_t* codes, const float* params, uint32_t units,
                              uint64_t tokens, uint32_t D, uint32_t bits, uint32_t G,
                              int per_channel, float* out, hipStream_t stream);
hipError_t launch_pytorch_order(const uint32_t* codes, uint32_t units, uint64_t tokens, uint32_t D,
                                uint32_t bits, uint32_t G, int per_channel, uint32_t* out,
                                hipStream_t stream);

// ---------------------------------------------------------------- attention (kernels_attn.hip)

// One decode-attention problem over a cache view plus an optional fp32 suffix per unit.
struct AttnProblem {
  CacheView cache;
  SeqState st;
  uint64_t seq;              // kq + kres  (= vq + vres)
  const float* suffix_k;     // [units][*][D] or null
  const float* suffix_v;
  uint64_t suffix_len;       // L
  uint64_t suffix_stride;    // floats between units of suffix_k / suffix_v
  const float* query;        // [batch][QH][D]
  float* out;                // [batch][QH][D]
  uint32_t qh;               // query heads
  uint32_t heads;            // kv heads
  uint32_t batch;
  float scale;
  // RuntimeKv::decode in one attention launch (null pend_k otherwise): `st` and `seq` already
  // count a decode token whose key and value rows are pend_k / pend_v ([units][D]). The merge
  // writes them to residual slot pend_kslot and window slot pend_vslot afterwards; with
  // pend_evict the token vq-1 left the window from slot pend_vslot and is quantized by the
  // attention launch. Needs the packed-chunk path (attention_fuses_decode).
  const float* pend_k;
  const float* pend_v;
  uint32_t pend_kslot, pend_vslot;
  uint32_t pend_evict;
};

// Whether launch_attention takes the packed-chunk path for p (the one that can carry a decode
// token appended in the same launch).
bool attention_fuses_decode(const AttnProblem& p);

// Workspace floats the attention needs for `p` (split-K partials).
size_t attention_workspace_floats(const AttnProblem& p);
hipError_t launch_attention(const AttnProblem& p, float* workspace, hipStream_t stream);

// Static attention workspace (kernels_attn.hip): a file-scope device array of
// kStaticWorkspaceFloats floats (8 MiB) that every device running the library holds until the
// process ends, for callers that cannot allocate. static_workspace gives its address on the
// current device, resolved once per device (hipGetSymbolAddress with that device current) and
// kept. Calls that use it share one array per device: calls that overlap on one device race.
constexpr size_t kStaticWorkspaceFloats = (size_t)2 << 20;
hipError_t static_workspace(float** out);

// out[0, n) = 0.f by a kernel (for callers that may capture the stream into a graph, where a
// memset node is avoided).
hipError_t launch_fill_zero(float* out, size_t n, hipStream_t stream);

// One session of a batched call: its fp32 suffix ([units][*][D], `stride` floats between
// units; k / v may be null when len is 0).
struct SessionDesc {
  const float* k;
  const float* v;
  uint64_t len;
  uint64_t stride;
};

// Sessions of one batched launch; larger batches run in groups of this many (each group
// streams the prefix once). Their descriptors travel in the kernel arguments (2 KB).
constexpr uint32_t kMaxLaunchSessions = 64;
struct SessionTable {
  SessionDesc d[kMaxLaunchSessions];
};

// n sessions sharing one prefix: each workgroup of the prefix's packed chunks serves every
// session in turn (the chunk data stays in L2 between sessions, so HBM sees the prefix once);
// the prefix window and each session's suffix run per session. Returns hipErrorNotSupported
// for shapes without the packed-chunk path (the caller then runs the sessions one by one).
struct SessionsProblem {
  CacheView cache;
  SeqState st;
  uint64_t seq;
  uint32_t n;
  const SessionDesc* sessions;  // host array of n (device suffix pointers)
  const float* queries;         // [n][batch][QH][D]
  float* out;                   // [n][batch][QH][D]
  uint32_t qh, heads, batch;
  float scale;
};
size_t sessions_workspace_floats(const SessionsProblem& p);
hipError_t launch_sessions_attention(const SessionsProblem& p, float* workspace,
                                     hipStream_t stream);

}  // namespace kivi
