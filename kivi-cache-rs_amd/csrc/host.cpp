// host.cpp — host state machine of the MI355X KIVI cache and the C ABI (include/kivi.h).
//
// Mirrors the reference's KiviCache / SharedPrefix / RagSession / RuntimeKv /
// QuantizedTensor (src/cache.rs, src/prefix.rs, src/runtime.rs, src/quant.rs) over device
// arenas: the packed streams, the key residual and the value window live in HBM and every
// transformation of KV data runs in the HIP kernels of kernels_*.hip. The host keeps only
// the counters (seq, kq, vq, residual lengths, ring head) and validates arguments in the
// reference's order. There is no CPU fallback: without a HIP device, entry points that
// touch data return KIVI_ERR_DEVICE.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <new>
#include <numeric>
#include <string>
#include <vector>

#include "kivi.h"
#include "common.hpp"

namespace kivi {
namespace {

// ---------------------------------------------------------------- status

struct Status {
  int code = KIVI_OK;
  uint64_t a = 0, b = 0;
  const char* name = nullptr;
  std::string detail;  // device errors
  bool ok() const { return code == KIVI_OK; }
};

Status Err(int code, uint64_t a = 0, uint64_t b = 0, const char* name = nullptr) {
  Status s;
  s.code = code;
  s.a = a;
  s.b = b;
  s.name = name;
  return s;
}

Status DevErr(hipError_t e, const char* what) {
  Status s = Err(KIVI_ERR_DEVICE);
  s.detail = std::string("HIP error in ") + what + ": " + hipGetErrorString(e);
  return s;
}

#define KIVI_TRY(expr)               \
  do {                               \
    Status _s = (expr);              \
    if (!_s.ok()) return _s;         \
  } while (0)

#define HIP_TRY(expr, what)                      \
  do {                                           \
    hipError_t _e = (expr);                      \
    if (_e != hipSuccess) return DevErr(_e, what); \
  } while (0)

// Display text of KiviError (src/error.rs:47-95) and of the extensions.
void format_error(const Status& s, kivi_error* e) {
  std::memset(e, 0, sizeof(*e));
  e->code = s.code;
  e->a = s.a;
  e->b = s.b;
  if (s.name != nullptr) std::snprintf(e->name, sizeof(e->name), "%s", s.name);
  char* m = e->message;
  const size_t n = sizeof(e->message);
  const unsigned long long A = s.a, B = s.b;
  switch (s.code) {
    case KIVI_ERR_INVALID_BITS:
      std::snprintf(m, n, "bit width %llu is not supported; use 2, 4, or 8", A);
      break;
    case KIVI_ERR_MISALIGNED_GROUP:
      std::snprintf(m, n, "group_size %llu * bits %llu must be a multiple of 32", A, B);
      break;
    case KIVI_ERR_RESIDUAL_LENGTH:
      std::snprintf(m, n, "residual_length %llu must be a positive multiple of group_size %llu", A, B);
      break;
    case KIVI_ERR_HEAD_DIM:
      std::snprintf(m, n, "head_dim %llu must be a positive multiple of group_size %llu", A, B);
      break;
    case KIVI_ERR_TOKEN_GROUP:
      std::snprintf(m, n,
                    "token count %llu must be a positive multiple of group_size %llu for "
                    "per-channel quantization",
                    A, B);
      break;
    case KIVI_ERR_ZERO_DIMENSION:
      std::snprintf(m, n, "%s must be greater than zero", s.name ? s.name : "?");
      break;
    case KIVI_ERR_SHAPE:
      std::snprintf(m, n, "expected %llu elements, got %llu", A, B);
      break;
    case KIVI_ERR_QUERY_HEADS:
      std::snprintf(m, n, "num_q_heads %llu must be a positive multiple of num_kv_heads %llu", A, B);
      break;
    case KIVI_ERR_NULL_ARGUMENT:
      std::snprintf(m, n, "%s must not be null", s.name ? s.name : "?");
      break;
    case KIVI_ERR_DEVICE:
      std::snprintf(m, n, "%s", s.detail.empty() ? "HIP device error" : s.detail.c_str());
      break;
    case KIVI_ERR_CAPACITY:
      if (s.name != nullptr)
        std::snprintf(m, n, "%s %llu exceeds the supported limit %llu", s.name, A, B);
      else
        std::snprintf(m, n, "size %llu exceeds the supported limit %llu", A, B);
      break;
    case KIVI_ERR_UNSUPPORTED:
      std::snprintf(m, n, "%s %llu is outside this build's limit %llu", s.name ? s.name : "value", A, B);
      break;
    case KIVI_ERR_MISMATCHED_PREFIX:
      std::snprintf(m, n, "session %llu does not share the first session's prefix", A);
      break;
    default:
      std::snprintf(m, n, "error %d", s.code);
      break;
  }
}

kivi_status report(const Status& s, kivi_error* err) {
  if (err != nullptr) {
    if (s.ok())
      std::memset(err, 0, sizeof(*err));
    else
      format_error(s, err);
  }
  return static_cast<kivi_status>(s.code);
}

template <class F>
kivi_status guarded(kivi_error* err, F&& f) {
  try {
    return report(f(), err);
  } catch (const std::bad_alloc&) {
    return report(Err(KIVI_ERR_CAPACITY, 0, 0), err);
  } catch (...) {
    Status s = Err(KIVI_ERR_DEVICE);
    s.detail = "unexpected exception";
    return report(s, err);
  }
}

Status need(const void* p, const char* name) {
  return p == nullptr ? Err(KIVI_ERR_NULL_ARGUMENT, 0, 0, name) : Status{};
}
// A null pointer is an empty slice only when the length is 0.
Status need_slice(const void* p, size_t len, const char* name) {
  return (p == nullptr && len != 0) ? Err(KIVI_ERR_NULL_ARGUMENT, 0, 0, name) : Status{};
}

// Checked products for shape arithmetic (the reference would overflow silently).
Status mul(size_t a, size_t b, size_t* out) {
  if (__builtin_mul_overflow(a, b, out)) return Err(KIVI_ERR_CAPACITY, a, SIZE_MAX / (b ? b : 1));
  return Status{};
}
Status mul4(size_t a, size_t b, size_t c, size_t d, size_t* out) {
  size_t x, y;
  KIVI_TRY(mul(a, b, &x));
  KIVI_TRY(mul(x, c, &y));
  return mul(y, d, out);
}

// ---------------------------------------------------------------- config checks

// check_bits_group (src/config.rs:47-55) and try_new (src/config.rs:31-45).
Status check_bits_group(uint8_t bits, size_t group_size) {
  if (!(bits == 2 || bits == 4 || bits == 8)) return Err(KIVI_ERR_INVALID_BITS, bits);
  if (group_size == 0 || (group_size * bits) % 32 != 0)
    return Err(KIVI_ERR_MISALIGNED_GROUP, group_size, bits);
  return Status{};
}
Status check_config(const kivi_config& c) {
  KIVI_TRY(check_bits_group(c.bits, c.group_size));
  if (c.residual_length == 0 || c.residual_length % c.group_size != 0)
    return Err(KIVI_ERR_RESIDUAL_LENGTH, c.residual_length, c.group_size);
  return Status{};
}

// Limits of this build (kernels index units and rows with 32-bit counters and stage one
// group / one 64-token value block per workgroup in LDS).
constexpr size_t kMaxHeadDim = 1024;
constexpr size_t kMaxKeyTile = 65536;       // G * D bytes of key codes staged per workgroup
constexpr size_t kMaxResidual = 1u << 20;
constexpr size_t kMaxUnits = (size_t)1 << 30;
constexpr size_t kMaxGqD = 8192;            // (num_q_heads/num_kv_heads) * head_dim

Status check_limits(const kivi_config& c, size_t batch, size_t heads, size_t head_dim) {
  if (head_dim > kMaxHeadDim) return Err(KIVI_ERR_UNSUPPORTED, head_dim, kMaxHeadDim, "head_dim");
  if (c.group_size * head_dim > kMaxKeyTile)
    return Err(KIVI_ERR_UNSUPPORTED, c.group_size * head_dim, kMaxKeyTile, "group_size*head_dim");
  if (c.residual_length > kMaxResidual)
    return Err(KIVI_ERR_UNSUPPORTED, c.residual_length, kMaxResidual, "residual_length");
  size_t units;
  KIVI_TRY(mul(batch, heads, &units));
  if (units > kMaxUnits) return Err(KIVI_ERR_UNSUPPORTED, units, kMaxUnits, "batch*num_kv_heads");
  return Status{};
}

// ---------------------------------------------------------------- device plumbing

int device_count() {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

Status current_device(int* dev) {
  if (device_count() <= 0) {
    Status s = Err(KIVI_ERR_DEVICE);
    s.detail = "no HIP device is available (the library has no CPU path)";
    return s;
  }
  HIP_TRY(hipGetDevice(dev), "hipGetDevice");
  return Status{};
}

// Makes `dev` current for the scope and restores the caller's device.
struct DeviceScope {
  int prev = -1;
  bool changed = false;
  explicit DeviceScope(int dev) {
    if (hipGetDevice(&prev) == hipSuccess && prev != dev) {
      changed = hipSetDevice(dev) == hipSuccess;
    }
  }
  ~DeviceScope() {
    if (changed) (void)hipSetDevice(prev);
  }
};

struct DevBuf {
  void* p = nullptr;
  size_t bytes = 0;
  DevBuf() = default;
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  ~DevBuf() { release(); }
  void release() {
    if (p != nullptr) (void)hipFree(p);
    p = nullptr;
    bytes = 0;
  }
  template <class T>
  T* as() const {
    return static_cast<T*>(p);
  }
  Status alloc_zero(size_t n, hipStream_t s, const char* what) {
    release();
    if (n == 0) return Status{};
    HIP_TRY(hipMalloc(&p, n), what);
    bytes = n;
    HIP_TRY(hipMemsetAsync(p, 0, n, s), what);
    return Status{};
  }
};

// Stream-ordered scratch for one call.
struct Scratch {
  void* p = nullptr;
  hipStream_t s = nullptr;
  ~Scratch() {
    if (p != nullptr) (void)hipFreeAsync(p, s);
  }
  Status get(size_t bytes, hipStream_t stream, const char* what) {
    s = stream;
    if (bytes == 0) return Status{};
    HIP_TRY(hipMallocAsync(&p, bytes, stream), what);
    return Status{};
  }
  template <class T>
  T* as() const {
    return static_cast<T*>(p);
  }
};

uint64_t lcm64(uint64_t a, uint64_t b) { return a / std::gcd(a, b) * b; }

// ---------------------------------------------------------------- cache state

struct CacheCore {
  kivi_config cfg{};
  size_t batch = 0, heads = 0, head_dim = 0;
  int device = 0;
  Geometry geo{};
  DevBuf kcodes, kparams, vcodes, vparams, kres, vring, smax;
  uint64_t seq = 0, kq = 0, vq = 0;
  uint32_t kres_len = 0, vres_len = 0, vhead = 0;
  hipStream_t stream = nullptr;

  uint32_t units() const { return geo.units; }
  uint64_t granule() const { return lcm64(kValueBlock, cfg.group_size); }

  CacheView view() const {
    CacheView v;
    v.geo = geo;
    v.kcodes = kcodes.as<uint32_t>();
    v.kparams = kparams.as<float>();
    v.vcodes = vcodes.as<uint32_t>();
    v.vparams = vparams.as<float>();
    v.kres = kres.as<float>();
    v.vring = vring.as<float>();
    v.smax = smax.as<uint32_t>();
    return v;
  }
  SeqState state() const {
    SeqState s;
    s.kq = kq;
    s.vq = vq;
    s.kres = kres_len;
    s.vres = vres_len;
    s.vhead = vhead;
    return s;
  }

  // Allocate residual buffers (src/cache.rs:105-119 preallocates them too).
  void set_geometry() {
    geo.bits = cfg.bits;
    geo.G = static_cast<uint32_t>(cfg.group_size);
    geo.R = static_cast<uint32_t>(cfg.residual_length);
    geo.D = static_cast<uint32_t>(head_dim);
    geo.units = static_cast<uint32_t>(batch * heads);
    geo.cap = 0;
  }

  // Packed capacity the arenas grow to when `tokens` must fit: at least double the current
  // capacity and 256 tokens, rounded up to the granule.
  uint64_t capacity_for(uint64_t tokens) const {
    const uint64_t gran = granule();
    uint64_t want = std::max<uint64_t>(tokens, geo.cap * 2);
    want = std::max<uint64_t>(want, 256);
    return (want + gran - 1) / gran * gran;
  }

  // Bytes of the packed arenas at the current capacity, the residual buffers and the maxima.
  size_t device_bytes() const {
    const size_t arenas = (geo.kcodes_unit() + geo.kparams_unit() + geo.vcodes_unit() +
                           geo.vparams_unit()) * geo.units * 4;
    return arenas + 2 * (size_t)geo.units * geo.R * geo.D * sizeof(float) +
           (size_t)geo.units * kMaxUnitWords * sizeof(uint32_t);
  }

  Status init(hipStream_t s) {
    set_geometry();
    const size_t rbytes = (size_t)geo.units * geo.R * geo.D * sizeof(float);
    KIVI_TRY(kres.alloc_zero(rbytes, s, "key residual"));
    KIVI_TRY(vring.alloc_zero(rbytes, s, "value window"));
    KIVI_TRY(smax.alloc_zero((size_t)geo.units * kMaxUnitWords * sizeof(uint32_t), s, "scale maxima"));
    return Status{};
  }

  // Grow the packed arenas to hold `tokens` per unit, keeping their contents.
  Status ensure_capacity(uint64_t tokens, hipStream_t s) {
    if (tokens <= geo.cap) return Status{};
    const uint64_t want = capacity_for(tokens);
    Geometry ng = geo;
    ng.cap = want;
    DevBuf nkc, nkp, nvc, nvp;
    KIVI_TRY(nkc.alloc_zero(ng.kcodes_unit() * ng.units * 4, s, "key codes"));
    KIVI_TRY(nkp.alloc_zero(ng.kparams_unit() * ng.units * 4, s, "key params"));
    KIVI_TRY(nvc.alloc_zero(ng.vcodes_unit() * ng.units * 4, s, "value codes"));
    KIVI_TRY(nvp.alloc_zero(ng.vparams_unit() * ng.units * 4, s, "value params"));
    if (geo.cap > 0) {
      HIP_TRY(copy_units(nkc.p, ng.kcodes_unit() * 4, kcodes.p, geo.kcodes_unit() * 4,
                         geo.kcodes_unit() * 4, geo.units, s), "grow key codes");
      HIP_TRY(copy_units(nkp.p, ng.kparams_unit() * 4, kparams.p, geo.kparams_unit() * 4,
                         geo.kparams_unit() * 4, geo.units, s), "grow key params");
      HIP_TRY(copy_units(nvc.p, ng.vcodes_unit() * 4, vcodes.p, geo.vcodes_unit() * 4,
                         geo.vcodes_unit() * 4, geo.units, s), "grow value codes");
      HIP_TRY(copy_units(nvp.p, ng.vparams_unit() * 4, vparams.p, geo.vparams_unit() * 4,
                         geo.vparams_unit() * 4, geo.units, s), "grow value params");
      HIP_TRY(hipStreamSynchronize(s), "grow");
    }
    std::swap(kcodes.p, nkc.p);
    std::swap(kcodes.bytes, nkc.bytes);
    std::swap(kparams.p, nkp.p);
    std::swap(kparams.bytes, nkp.bytes);
    std::swap(vcodes.p, nvc.p);
    std::swap(vcodes.bytes, nvc.bytes);
    std::swap(vparams.p, nvp.p);
    std::swap(vparams.bytes, nvp.bytes);
    geo.cap = want;
    return Status{};
  }

  // KiviCache::append on device rows (src/cache.rs:186-214, append_keys :382-430,
  // append_values :432-484). keys/values are [units][n][D] device arrays.
  Status append_rows(const float* keys, const float* values, uint64_t n, hipStream_t s) {
    if (n == 0) return Status{};
    const uint64_t R = cfg.residual_length, G = cfg.group_size, D = head_dim;
    const uint64_t kq_after = kq + ((kres_len + n) / R) * R;
    const uint64_t total = seq + n;
    const uint64_t vq_after = total > R ? total - R : 0;
    KIVI_TRY(ensure_capacity(std::max(kq_after, vq_after), s));
    const CacheView cv = view();
    // one decode token: residual copy, window eviction and window write in one launch
    if (n == 1 && vres_len <= R) {
      const bool evict = vres_len == R;
      const uint32_t vslot = evict ? vhead : static_cast<uint32_t>((vhead + vres_len) % R);
      const hipError_t e = launch_decode_append(cv, keys, values, kres_len, vslot, evict, vq, s);
      if (e == hipSuccess) {
        kres_len += 1;
        if (kres_len == R) {
          HIP_TRY(launch_quant_keys(cv, RowSource{cv.kres, R * D, 0, 0}, kq / G,
                                    static_cast<uint32_t>(R / G), s), "key flush");
          kq += R;
          kres_len = 0;
        }
        if (evict) {
          vq += 1;
          vhead = static_cast<uint32_t>((vhead + 1) % R);
        } else {
          vres_len += 1;
        }
        seq += 1;
        return Status{};
      }
      // hipErrorNotSupported: a shape the one-launch append does not cover, refused before
      // any launch (so HIP's last-error state is untouched); the general path below runs
      if (e != hipErrorNotSupported) HIP_TRY(e, "decode append");
    }
    const RowSource kin{keys, n * D, 0, 0};
    // ---- keys: fill the residual, flush every R tokens, quantize whole R-blocks of the
    // input in place (the same groups the reference forms by copy-then-flush).
    uint64_t off = 0;
    if (kres_len > 0) {
      const uint64_t take = std::min<uint64_t>(R - kres_len, n);
      HIP_TRY(launch_copy_rows(geo, RowSource{keys, n * D, 0, 0}, cv.kres, kres_len,
                               static_cast<uint32_t>(take), s), "key residual copy");
      kres_len += static_cast<uint32_t>(take);
      off = take;
      if (kres_len == R) {
        HIP_TRY(launch_quant_keys(cv, RowSource{cv.kres, R * D, 0, 0}, kq / G,
                                  static_cast<uint32_t>(R / G), s), "key flush");
        kq += R;
        kres_len = 0;
      }
    }
    const uint64_t full = (n - off) / R;
    if (full > 0) {
      RowSource src = kin;
      src.offset = off;
      const uint64_t groups = full * R / G;
      // keep one launch's grid within 2^31 workgroups
      uint64_t done = 0;
      while (done < groups) {
        const uint64_t chunk = std::min<uint64_t>(groups - done, (1u << 30) / std::max<uint32_t>(geo.units, 1));
        RowSource sc = src;
        sc.offset = off + done * G;
        HIP_TRY(launch_quant_keys(cv, sc, kq / G + done, static_cast<uint32_t>(chunk), s), "key quantize");
        done += chunk;
      }
      kq += full * R;
      off += full * R;
    }
    const uint64_t rem = n - off;
    if (rem > 0) {
      HIP_TRY(launch_copy_rows(geo, RowSource{keys, n * D, off, 0}, cv.kres, kres_len,
                               static_cast<uint32_t>(rem), s), "key residual copy");
      kres_len += static_cast<uint32_t>(rem);
    }
    // ---- values: sliding window of R tokens kept as a ring.
    const RowSource ring{cv.vring, R * D, vhead, 1};
    if (n >= R) {
      const uint64_t quant_n = n - R;
      HIP_TRY(launch_quant_values(cv, ring, vres_len, RowSource{values, n * D, 0, 0}, quant_n, vq, s),
              "value quantize");
      vq += vres_len + quant_n;
      HIP_TRY(launch_copy_rows(geo, RowSource{values, n * D, quant_n, 0}, cv.vring, 0,
                               static_cast<uint32_t>(R), s), "value window copy");
      vhead = 0;
      vres_len = static_cast<uint32_t>(R);
    } else {
      const uint64_t combined = vres_len + n;
      const uint64_t drop = combined > R ? combined - R : 0;
      if (drop > 0) {
        HIP_TRY(launch_quant_values(cv, ring, static_cast<uint32_t>(drop), RowSource{nullptr, 0, 0, 0}, 0, vq, s),
                "value evict");
        vq += drop;
        vhead = static_cast<uint32_t>((vhead + drop) % R);
        vres_len -= static_cast<uint32_t>(drop);
      }
      HIP_TRY(launch_copy_rows(geo, RowSource{values, n * D, 0, 0}, cv.vring,
                               static_cast<uint32_t>((vhead + vres_len) % R), static_cast<uint32_t>(n), s),
              "value window copy");
      vres_len += static_cast<uint32_t>(n);
    }
    seq += n;
    return Status{};
  }

  // KiviCache::memory (src/cache.rs:362-380) from the counters.
  kivi_memory_report memory() const {
    kivi_memory_report r{};
    const size_t u = units(), D = head_dim, G = cfg.group_size, b = cfg.bits;
    r.tokens = seq;
    r.key_code_bytes = u * kq * D * b / 8;
    r.key_metadata_bytes = u * (kq / G) * D * 2 * 4;
    r.value_code_bytes = u * vq * D * b / 8;
    r.value_metadata_bytes = u * vq * (D / G) * 2 * 4;
    const size_t elements = u * D;
    r.key_residual_bytes = (size_t)kres_len * elements * 4;
    r.value_residual_bytes = (size_t)vres_len * elements * 4;
    r.residual_capacity_bytes = 2 * cfg.residual_length * elements * 4;
    r.fp16_baseline_bytes = 2 * seq * elements * 2;
    r.fp32_baseline_bytes = 2 * seq * elements * 4;
    return r;
  }

  // Deep copy for SharedPrefix::from_cache (src/prefix.rs:74-92); the copy's arenas are
  // sized to the frozen length.
  Status copy_into(CacheCore& dst, hipStream_t s) const {
    dst.cfg = cfg;
    dst.batch = batch;
    dst.heads = heads;
    dst.head_dim = head_dim;
    dst.device = device;
    dst.seq = seq;
    dst.kq = kq;
    dst.vq = vq;
    dst.kres_len = kres_len;
    dst.vres_len = vres_len;
    dst.vhead = vhead;
    KIVI_TRY(dst.init(s));
    const size_t rbytes = (size_t)geo.units * geo.R * geo.D * sizeof(float);
    HIP_TRY(hipMemcpyAsync(dst.kres.p, kres.p, rbytes, hipMemcpyDeviceToDevice, s), "prefix copy");
    HIP_TRY(hipMemcpyAsync(dst.vring.p, vring.p, rbytes, hipMemcpyDeviceToDevice, s), "prefix copy");
    HIP_TRY(hipMemcpyAsync(dst.smax.p, smax.p, smax.bytes, hipMemcpyDeviceToDevice, s), "prefix copy");
    const uint64_t used = std::max(kq, vq);
    if (used > 0) {
      const uint64_t gran = granule();
      Geometry ng = geo;
      ng.cap = (used + gran - 1) / gran * gran;
      KIVI_TRY(dst.kcodes.alloc_zero(ng.kcodes_unit() * ng.units * 4, s, "prefix key codes"));
      KIVI_TRY(dst.kparams.alloc_zero(ng.kparams_unit() * ng.units * 4, s, "prefix key params"));
      KIVI_TRY(dst.vcodes.alloc_zero(ng.vcodes_unit() * ng.units * 4, s, "prefix value codes"));
      KIVI_TRY(dst.vparams.alloc_zero(ng.vparams_unit() * ng.units * 4, s, "prefix value params"));
      HIP_TRY(copy_units(dst.kcodes.p, ng.kcodes_unit() * 4, kcodes.p, geo.kcodes_unit() * 4,
                         ng.kcodes_unit() * 4, geo.units, s), "prefix copy");
      HIP_TRY(copy_units(dst.kparams.p, ng.kparams_unit() * 4, kparams.p, geo.kparams_unit() * 4,
                         ng.kparams_unit() * 4, geo.units, s), "prefix copy");
      HIP_TRY(copy_units(dst.vcodes.p, ng.vcodes_unit() * 4, vcodes.p, geo.vcodes_unit() * 4,
                         ng.vcodes_unit() * 4, geo.units, s), "prefix copy");
      HIP_TRY(copy_units(dst.vparams.p, ng.vparams_unit() * 4, vparams.p, geo.vparams_unit() * 4,
                         ng.vparams_unit() * 4, geo.units, s), "prefix copy");
      dst.geo.cap = ng.cap;
    }
    return Status{};
  }
};

size_t compressed_bytes(const kivi_memory_report& r) {
  return r.key_code_bytes + r.key_metadata_bytes + r.value_code_bytes + r.value_metadata_bytes +
         r.key_residual_bytes + r.value_residual_bytes;
}

// Workspace of one attention target (a cache or a session). Two calls sharing it must not
// overlap on the device: calls on one stream are ordered by the stream; when a call comes on
// another stream, an event recorded at that moment on the previous call's stream is waited
// for first (no per-call event, which would stall the queue).
struct AttnSync {
  DevBuf workspace;  // split partials, grown on demand
  hipEvent_t done = nullptr;
  bool used = false;
  hipStream_t last = nullptr;
  std::mutex mu;
  AttnSync() = default;
  AttnSync(const AttnSync&) = delete;
  AttnSync& operator=(const AttnSync&) = delete;
  ~AttnSync() {
    if (done != nullptr) (void)hipEventDestroy(done);
  }
  Status init() {
    HIP_TRY(hipEventCreateWithFlags(&done, hipEventDisableTiming), "attention event");
    return Status{};
  }
  Status before(hipStream_t s) {
    if (used && s != last) {
      HIP_TRY(hipEventRecord(done, last), "attention ordering");
      HIP_TRY(hipStreamWaitEvent(s, done, 0), "attention ordering");
    }
    return Status{};
  }
  Status after(hipStream_t s) {
    used = true;
    last = s;
    return Status{};
  }
  // Waits until the last call's work is done (before freeing or regrowing).
  Status drain() {
    if (used) HIP_TRY(hipStreamSynchronize(last), "attention drain");
    return Status{};
  }
  // Workspace of at least `bytes`; growing waits for the previous call to finish with it.
  Status reserve(size_t bytes) {
    if (bytes <= workspace.bytes) return Status{};
    KIVI_TRY(drain());
    workspace.release();
    HIP_TRY(hipMalloc(&workspace.p, bytes), "attention workspace");
    workspace.bytes = bytes;
    return Status{};
  }
};

// The attention problem over `core` plus an optional device suffix (tape_only: the suffix
// rows alone), after the limit check every attention entry point shares.
Status attention_problem(const CacheCore& core, const float* suffix_k, const float* suffix_v,
                         uint64_t L, uint64_t suffix_stride, const float* query, size_t qh,
                         float scale, float* out, bool tape_only, AttnProblem* out_p) {
  const size_t gq = qh / core.heads;
  if (gq * core.head_dim > kMaxGqD)
    return Err(KIVI_ERR_UNSUPPORTED, gq * core.head_dim, kMaxGqD, "(num_q_heads/num_kv_heads)*head_dim");
  const uint64_t seq = tape_only ? 0 : core.seq;
  AttnProblem& p = *out_p;
  p = AttnProblem{};
  p.cache = core.view();
  p.st = tape_only ? SeqState{} : core.state();
  p.seq = seq;
  p.suffix_k = suffix_k;
  p.suffix_v = suffix_v;
  p.suffix_len = L;
  p.suffix_stride = suffix_stride;
  p.query = query;
  p.out = out;
  p.qh = static_cast<uint32_t>(qh);
  p.heads = static_cast<uint32_t>(core.heads);
  p.batch = static_cast<uint32_t>(core.batch);
  p.scale = scale;
  return Status{};
}

// Attention over `core` plus an optional device suffix, writing `out` on the device.
// With `tape_only` the cache's tokens are left out: attention over the suffix rows alone
// (the QualityGuard's fp32 attention over its tape).
Status attend(const CacheCore& core, AttnSync& sync, const float* suffix_k, const float* suffix_v,
              uint64_t L, uint64_t suffix_stride, const float* query, size_t qh, float scale,
              float* out, hipStream_t s, bool tape_only = false) {
  AttnProblem p;
  KIVI_TRY(attention_problem(core, suffix_k, suffix_v, L, suffix_stride, query, qh, scale, out, tape_only, &p));
  if (p.seq + L == 0) {
    HIP_TRY(hipMemsetAsync(out, 0, core.batch * qh * core.head_dim * sizeof(float), s), "attention zero output");
    return Status{};
  }
  std::lock_guard<std::mutex> lock(sync.mu);
  KIVI_TRY(sync.reserve(attention_workspace_floats(p) * sizeof(float)));
  KIVI_TRY(sync.before(s));
  HIP_TRY(launch_attention(p, sync.workspace.as<float>(), s), "attention");
  KIVI_TRY(sync.after(s));
  return Status{};
}

// Shape checks of KiviCache::attention (src/cache.rs:230-242), then the out buffer.
Status check_attention(size_t batch, size_t heads, size_t head_dim, size_t query_len,
                       size_t num_q_heads, size_t out_len) {
  if (num_q_heads == 0 || num_q_heads % heads != 0)
    return Err(KIVI_ERR_QUERY_HEADS, num_q_heads, heads);
  size_t expected;
  KIVI_TRY(mul4(batch, num_q_heads, head_dim, 1, &expected));
  if (query_len != expected) return Err(KIVI_ERR_SHAPE, expected, query_len);
  if (out_len != expected) return Err(KIVI_ERR_SHAPE, expected, out_len);
  return Status{};
}

Status sync(hipStream_t s, const char* what) {
  HIP_TRY(hipStreamSynchronize(s), what);
  HIP_TRY(hipGetLastError(), what);
  return Status{};
}

}  // namespace
}  // namespace kivi

using namespace kivi;

// ---------------------------------------------------------------- opaque handles

// The stream of the latest device-pointer call on a cache or session, whose work may still run
// there. The host-pointer calls return complete, as the reference's calls do: before they
// enqueue on their own stream they wait for that stream when it is another one (settle), so
// they never overlap its work.
struct DeviceCallOrder {
  std::mutex mu;
  hipStream_t stream = nullptr;
  bool pending = false;
  void note(hipStream_t s) {
    std::lock_guard<std::mutex> lock(mu);
    stream = s;
    pending = true;
  }
  Status settle(hipStream_t own) {
    std::lock_guard<std::mutex> lock(mu);
    if (pending && stream != own) {
      // a stream still capturing holds no work yet (its graph runs where it is launched)
      hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
      HIP_TRY(hipStreamIsCapturing(stream, &cs), "device-call ordering");
      if (cs == hipStreamCaptureStatusNone) HIP_TRY(hipStreamSynchronize(stream), "device-call ordering");
    }
    pending = false;
    return Status{};
  }
};

struct kivi_cache {
  CacheCore core;
  AttnSync attn;
  std::mutex mu;  // one mutating call at a time (the reference's &mut self)
  DeviceCallOrder dev;  // host-pointer calls work on core.stream; freeing waits too
  void note_device(hipStream_t s) { dev.note(s); }
  Status settle() { return dev.settle(core.stream); }
};

struct kivi_prefix_state {
  CacheCore core;
  size_t prefix_bytes = 0;
  mutable AttnSync batch;  // workspace of batched session calls over this prefix
};

struct kivi_prefix {
  std::shared_ptr<kivi_prefix_state> state;  // SharedPrefix = Arc<PrefixState>
  std::atomic<int> refs{1};
};

struct kivi_session {
  kivi_prefix* prefix = nullptr;  // holds one reference
  AttnSync attn;
  DevBuf keys, values;            // [units][cap][D] fp32 suffix (the reference re-splices, src/prefix.rs:196-221)
  uint64_t len = 0, cap = 0;
  DeviceCallOrder dev;            // host-pointer calls work on the default stream
};

struct kivi_runtime {
  kivi_cache cache;
};

struct kivi_quantized {
  int device = 0;
  int axis = 0;
  uint8_t bits = 0;
  size_t group_size = 0, batch = 0, heads = 0, tokens = 0, head_dim = 0;
  DevBuf codes, params;  // reference PackedStream order, concatenated over units
  size_t n_codes = 0, n_params = 0;
  mutable DeviceCallOrder dev;  // the stream of a `*_device` quantize; host reads wait for it
  kivi_quantized() = default;
  kivi_quantized(const kivi_quantized&) = delete;
  kivi_quantized& operator=(const kivi_quantized&) = delete;
};

namespace {

Status create_cache(const kivi_config* config, size_t batch, size_t heads, size_t head_dim,
                    kivi_cache* c) {
  KIVI_TRY(need(config, "config"));
  KIVI_TRY(check_config(*config));
  // KiviCache::new check order (src/cache.rs:93-104).
  if (batch == 0) return Err(KIVI_ERR_ZERO_DIMENSION, 0, 0, "batch");
  if (heads == 0) return Err(KIVI_ERR_ZERO_DIMENSION, 0, 0, "num_kv_heads");
  if (head_dim == 0 || head_dim % config->group_size != 0)
    return Err(KIVI_ERR_HEAD_DIM, head_dim, config->group_size);
  KIVI_TRY(check_limits(*config, batch, heads, head_dim));
  int dev = 0;
  KIVI_TRY(current_device(&dev));
  c->core.cfg = *config;
  c->core.batch = batch;
  c->core.heads = heads;
  c->core.head_dim = head_dim;
  c->core.device = dev;
  KIVI_TRY(c->core.init(nullptr));
  KIVI_TRY(c->attn.init());
  return sync(nullptr, "cache init");
}

Status cache_append(kivi_cache* c, const float* keys, size_t keys_len, const float* values,
                    size_t values_len, size_t seq_len, bool device, hipStream_t stream) {
  KIVI_TRY(need(c, "cache"));
  CacheCore& core = c->core;
  size_t expected;
  KIVI_TRY(mul4(core.batch, core.heads, seq_len, core.head_dim, &expected));
  if (keys_len != expected) return Err(KIVI_ERR_SHAPE, expected, keys_len);
  if (values_len != expected) return Err(KIVI_ERR_SHAPE, expected, values_len);
  if (seq_len == 0) return Status{};
  KIVI_TRY(need_slice(keys, keys_len, "keys"));
  KIVI_TRY(need_slice(values, values_len, "values"));
  std::lock_guard<std::mutex> lock(c->mu);
  DeviceScope scope(core.device);
  if (device) return core.append_rows(keys, values, seq_len, stream);
  hipStream_t s = core.stream;
  Scratch dk, dv;
  KIVI_TRY(dk.get(expected * 4, s, "append staging"));
  KIVI_TRY(dv.get(expected * 4, s, "append staging"));
  HIP_TRY(hipMemcpyAsync(dk.p, keys, expected * 4, hipMemcpyHostToDevice, s), "append H2D");
  HIP_TRY(hipMemcpyAsync(dv.p, values, expected * 4, hipMemcpyHostToDevice, s), "append H2D");
  KIVI_TRY(core.append_rows(dk.as<float>(), dv.as<float>(), seq_len, s));
  return sync(s, "append");
}

Status cache_attention(const kivi_cache* c, const float* query, size_t query_len,
                       size_t num_q_heads, float scale, float* out, size_t out_len, bool device,
                       hipStream_t stream) {
  KIVI_TRY(need(c, "cache"));
  const CacheCore& core = c->core;
  KIVI_TRY(check_attention(core.batch, core.heads, core.head_dim, query_len, num_q_heads, out_len));
  KIVI_TRY(need_slice(query, query_len, "query"));
  KIVI_TRY(need_slice(out, out_len, "out"));
  DeviceScope scope(core.device);
  kivi_cache* mc = const_cast<kivi_cache*>(c);  // its workspace only; the cache itself is read
  if (device) return attend(core, mc->attn, nullptr, nullptr, 0, 0, query, num_q_heads, scale, out, stream);
  hipStream_t s = core.stream;
  Scratch dq, dout;
  KIVI_TRY(dq.get(query_len * 4, s, "attention staging"));
  KIVI_TRY(dout.get(out_len * 4, s, "attention staging"));
  HIP_TRY(hipMemcpyAsync(dq.p, query, query_len * 4, hipMemcpyHostToDevice, s), "attention H2D");
  KIVI_TRY(attend(core, mc->attn, nullptr, nullptr, 0, 0, dq.as<float>(), num_q_heads, scale,
                  dout.as<float>(), s));
  HIP_TRY(hipMemcpyAsync(out, dout.p, out_len * 4, hipMemcpyDeviceToHost, s), "attention D2H");
  return sync(s, "attention");
}

// Ordering of the calls that share one device's static workspace. Calls on one stream are
// ordered by the stream. An eager call on another stream than the previous eager call first
// waits for an event recorded on that stream at this moment (as AttnSync does for a cache's
// own workspace). The event is created once per device, with the workspace's address, at the
// first call there. A call enqueued under stream capture is ordered only by the stream its
// graph is later launched on, and leaves the eager ordering state alone.
struct StaticWorkspaceSlot {
  std::mutex mu;
  float* ws = nullptr;
  hipEvent_t done = nullptr;
  hipStream_t last = nullptr;
  bool used = false;
};
constexpr int kMaxStaticDevices = 64;
std::mutex g_static_mu;
StaticWorkspaceSlot g_static_slots[kMaxStaticDevices];

Status static_workspace_slot(int device, StaticWorkspaceSlot** out) {
  if (device < 0 || device >= kMaxStaticDevices)
    return Err(KIVI_ERR_UNSUPPORTED, static_cast<size_t>(device), kMaxStaticDevices, "device index");
  std::lock_guard<std::mutex> lock(g_static_mu);
  StaticWorkspaceSlot& slot = g_static_slots[device];
  if (slot.ws == nullptr) {
    float* ws = nullptr;
    HIP_TRY(static_workspace(&ws), "static attention workspace");
    HIP_TRY(hipEventCreateWithFlags(&slot.done, hipEventDisableTiming), "static workspace event");
    slot.ws = ws;
  }
  *out = &slot;
  return Status{};
}

// KiviCache::attention on device pointers with the split partials in the library's static
// per-device workspace: no allocation, no memset (an empty cache's zeros come from a fill
// kernel), no host-side wait. Checks as cache_attention, then the workspace size. Eager calls
// on different streams are ordered by StaticWorkspaceSlot; calls on one stream by the stream.
Status cache_attention_noalloc(const kivi_cache* c, const float* query, size_t query_len,
                               size_t num_q_heads, float scale, float* out, size_t out_len,
                               hipStream_t stream) {
  KIVI_TRY(need(c, "cache"));
  const CacheCore& core = c->core;
  KIVI_TRY(check_attention(core.batch, core.heads, core.head_dim, query_len, num_q_heads, out_len));
  KIVI_TRY(need_slice(query, query_len, "query"));
  KIVI_TRY(need_slice(out, out_len, "out"));
  DeviceScope scope(core.device);
  AttnProblem p;
  KIVI_TRY(attention_problem(core, nullptr, nullptr, 0, 0, query, num_q_heads, scale, out, false, &p));
  if (p.seq == 0) {
    HIP_TRY(launch_fill_zero(out, out_len, stream), "attention zero output");
    return Status{};
  }
  const size_t floats = attention_workspace_floats(p);
  if (floats > kStaticWorkspaceFloats)
    return Err(KIVI_ERR_CAPACITY, floats, kStaticWorkspaceFloats, "attention workspace floats");
  StaticWorkspaceSlot* slot = nullptr;
  KIVI_TRY(static_workspace_slot(core.device, &slot));
  std::lock_guard<std::mutex> lock(slot->mu);
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  HIP_TRY(hipStreamIsCapturing(stream, &capture), "attention capture status");
  const bool eager = capture == hipStreamCaptureStatusNone;
  if (eager && slot->used && slot->last != stream) {
    HIP_TRY(hipEventRecord(slot->done, slot->last), "static workspace ordering");
    HIP_TRY(hipStreamWaitEvent(stream, slot->done, 0), "static workspace ordering");
  }
  HIP_TRY(launch_attention(p, slot->ws, stream), "attention");
  if (eager) {
    slot->used = true;
    slot->last = stream;
  }
  return Status{};
}

// KiviCache::dequantize (src/cache.rs:282-325) into host buffers (staged) or device buffers.
Status cache_dequantize(const kivi_cache* cache, float* keys, size_t keys_len, float* values,
                        size_t values_len, bool device, hipStream_t stream) {
  KIVI_TRY(need(cache, "cache"));
  const CacheCore& core = cache->core;
  size_t n;
  KIVI_TRY(mul4(core.batch, core.heads, core.seq, core.head_dim, &n));
  if (keys_len != n) return Err(KIVI_ERR_SHAPE, n, keys_len);
  if (values_len != n) return Err(KIVI_ERR_SHAPE, n, values_len);
  if (n == 0) return Status{};
  KIVI_TRY(need(keys, "keys"));
  KIVI_TRY(need(values, "values"));
  DeviceScope scope(core.device);
  if (device) {
    HIP_TRY(launch_dequant_cache(core.view(), core.state(), keys, values, stream), "dequantize");
    return Status{};
  }
  hipStream_t s = core.stream;
  Scratch dk, dv;
  KIVI_TRY(dk.get(n * 4, s, "dequantize"));
  KIVI_TRY(dv.get(n * 4, s, "dequantize"));
  HIP_TRY(launch_dequant_cache(core.view(), core.state(), dk.as<float>(), dv.as<float>(), s), "dequantize");
  HIP_TRY(hipMemcpyAsync(keys, dk.p, n * 4, hipMemcpyDeviceToHost, s), "dequantize D2H");
  HIP_TRY(hipMemcpyAsync(values, dv.p, n * 4, hipMemcpyDeviceToHost, s), "dequantize D2H");
  return sync(s, "dequantize");
}

// Packed streams in the reference PackedStream order, into host (staged) or device buffers;
// a NULL array is skipped.
Status cache_export(const kivi_cache* cache, uint32_t* key_codes, size_t key_codes_len,
                    float* key_params, size_t key_params_len, uint32_t* value_codes,
                    size_t value_codes_len, float* value_params, size_t value_params_len,
                    bool device, hipStream_t stream) {
  KIVI_TRY(need(cache, "cache"));
  const CacheCore& core = cache->core;
  const size_t u = core.units(), D = core.head_dim, G = core.cfg.group_size;
  const size_t nkc = u * core.kq * D / (32 / core.cfg.bits);
  const size_t nkp = u * (core.kq / G) * D * 2;
  const size_t nvc = u * core.vq * D / (32 / core.cfg.bits);
  const size_t nvp = u * core.vq * (D / G) * 2;
  if (key_codes && key_codes_len != nkc) return Err(KIVI_ERR_SHAPE, nkc, key_codes_len);
  if (key_params && key_params_len != nkp) return Err(KIVI_ERR_SHAPE, nkp, key_params_len);
  if (value_codes && value_codes_len != nvc) return Err(KIVI_ERR_SHAPE, nvc, value_codes_len);
  if (value_params && value_params_len != nvp) return Err(KIVI_ERR_SHAPE, nvp, value_params_len);
  DeviceScope scope(core.device);
  const CacheView cv = core.view();
  if (device) {
    HIP_TRY(launch_export_keys(cv, core.kq, nkc ? key_codes : nullptr, nkp ? key_params : nullptr, stream),
            "export keys");
    HIP_TRY(launch_export_values(cv, core.vq, nvc ? value_codes : nullptr, nvp ? value_params : nullptr,
                                 stream), "export values");
    return Status{};
  }
  hipStream_t s = core.stream;
  Scratch a, b, c, d;
  if (key_codes && nkc) KIVI_TRY(a.get(nkc * 4, s, "export"));
  if (key_params && nkp) KIVI_TRY(b.get(nkp * 4, s, "export"));
  if (value_codes && nvc) KIVI_TRY(c.get(nvc * 4, s, "export"));
  if (value_params && nvp) KIVI_TRY(d.get(nvp * 4, s, "export"));
  HIP_TRY(launch_export_keys(cv, core.kq, a.as<uint32_t>(), b.as<float>(), s), "export keys");
  HIP_TRY(launch_export_values(cv, core.vq, c.as<uint32_t>(), d.as<float>(), s), "export values");
  if (a.p) HIP_TRY(hipMemcpyAsync(key_codes, a.p, nkc * 4, hipMemcpyDeviceToHost, s), "export D2H");
  if (b.p) HIP_TRY(hipMemcpyAsync(key_params, b.p, nkp * 4, hipMemcpyDeviceToHost, s), "export D2H");
  if (c.p) HIP_TRY(hipMemcpyAsync(value_codes, c.p, nvc * 4, hipMemcpyDeviceToHost, s), "export D2H");
  if (d.p) HIP_TRY(hipMemcpyAsync(value_params, d.p, nvp * 4, hipMemcpyDeviceToHost, s), "export D2H");
  return sync(s, "export");
}

// RuntimeKv::decode on device pointers in one attention launch plus its merge: the attention
// reads the new token's rows from the inputs, quantizes the token the window evicts, and the
// merge writes the rows to the residual and the window (src/runtime.rs:46-56 = append(key,
// value, 1) then attention, bit for bit). Taken when both calls' checks pass, no key flush is
// due and the attention runs on the packed-chunk path; *fused is false otherwise (nothing
// done), and the caller appends and attends in two calls.
Status decode_fused(kivi_cache* c, const float* key, size_t key_len, const float* value,
                    size_t value_len, const float* query, size_t query_len, size_t num_q_heads,
                    float scale, float* out, size_t out_len, hipStream_t s, bool* fused) {
  *fused = false;
  if (c == nullptr) return Status{};
  CacheCore& core = c->core;
  size_t expected;
  if (!mul4(core.batch, core.heads, 1, core.head_dim, &expected).ok() || key_len != expected ||
      value_len != expected || key == nullptr || value == nullptr)
    return Status{};
  if (!check_attention(core.batch, core.heads, core.head_dim, query_len, num_q_heads, out_len).ok() ||
      query == nullptr || out == nullptr)
    return Status{};
  std::lock_guard<std::mutex> lock(c->mu);
  const uint32_t R = static_cast<uint32_t>(core.cfg.residual_length);
  if (core.kres_len + 1 >= R || core.vres_len > R) return Status{};  // a key flush is due
  const bool evict = core.vres_len == R;
  AttnProblem p{};
  p.cache = core.view();
  p.st = core.state();
  p.st.kres += 1;
  if (evict) {
    p.st.vq += 1;
    p.st.vhead = (p.st.vhead + 1) % R;
  } else {
    p.st.vres += 1;
  }
  p.seq = core.seq + 1;
  p.query = query;
  p.out = out;
  p.qh = static_cast<uint32_t>(num_q_heads);
  p.heads = static_cast<uint32_t>(core.heads);
  p.batch = static_cast<uint32_t>(core.batch);
  p.scale = scale;
  p.pend_k = key;
  p.pend_v = value;
  p.pend_kslot = core.kres_len;
  p.pend_vslot = evict ? core.vhead : (core.vhead + core.vres_len) % R;
  p.pend_evict = evict ? 1u : 0u;
  if (!attention_fuses_decode(p)) return Status{};
  DeviceScope scope(core.device);
  KIVI_TRY(core.ensure_capacity(p.st.vq, s));
  p.cache = core.view();  // capacity growth moves the arrays
  std::lock_guard<std::mutex> alock(c->attn.mu);
  KIVI_TRY(c->attn.reserve(attention_workspace_floats(p) * sizeof(float)));
  KIVI_TRY(c->attn.before(s));
  HIP_TRY(launch_attention(p, c->attn.workspace.as<float>(), s), "decode attention");
  KIVI_TRY(c->attn.after(s));
  core.kres_len += 1;
  if (evict) {
    core.vq += 1;
    core.vhead = p.st.vhead;
  } else {
    core.vres_len += 1;
  }
  core.seq += 1;
  *fused = true;
  return Status{};
}

Status session_attend(const kivi_session* se, const float* query, size_t query_len,
                      size_t num_q_heads, float scale, float* out, size_t out_len, bool device,
                      hipStream_t stream) {
  KIVI_TRY(need(se, "session"));
  const CacheCore& core = se->prefix->state->core;
  KIVI_TRY(check_attention(core.batch, core.heads, core.head_dim, query_len, num_q_heads, out_len));
  KIVI_TRY(need_slice(query, query_len, "query"));
  KIVI_TRY(need_slice(out, out_len, "out"));
  DeviceScope scope(core.device);
  const uint64_t stride = se->cap * core.head_dim;
  kivi_session* ms = const_cast<kivi_session*>(se);  // its workspace only
  if (device)
    return attend(core, ms->attn, se->keys.as<float>(), se->values.as<float>(), se->len, stride,
                  query, num_q_heads, scale, out, stream);
  hipStream_t s = nullptr;
  Scratch dq, dout;
  KIVI_TRY(dq.get(query_len * 4, s, "attention staging"));
  KIVI_TRY(dout.get(out_len * 4, s, "attention staging"));
  HIP_TRY(hipMemcpyAsync(dq.p, query, query_len * 4, hipMemcpyHostToDevice, s), "attention H2D");
  KIVI_TRY(attend(core, ms->attn, se->keys.as<float>(), se->values.as<float>(), se->len, stride,
                  dq.as<float>(), num_q_heads, scale, dout.as<float>(), s));
  HIP_TRY(hipMemcpyAsync(out, dout.p, out_len * 4, hipMemcpyDeviceToHost, s), "attention D2H");
  return sync(s, "session attention");
}

// RagSession::append (src/prefix.rs:173-223) into a capacity-managed device suffix.
Status session_append(kivi_session* se, const float* keys, size_t keys_len, const float* values,
                      size_t values_len, size_t seq_len, bool device, hipStream_t stream) {
  KIVI_TRY(need(se, "session"));
  const CacheCore& core = se->prefix->state->core;
  size_t expected;
  KIVI_TRY(mul4(core.batch, core.heads, seq_len, core.head_dim, &expected));
  if (keys_len != expected) return Err(KIVI_ERR_SHAPE, expected, keys_len);
  if (values_len != expected) return Err(KIVI_ERR_SHAPE, expected, values_len);
  if (seq_len == 0) return Status{};
  KIVI_TRY(need_slice(keys, keys_len, "keys"));
  KIVI_TRY(need_slice(values, values_len, "values"));
  DeviceScope scope(core.device);
  hipStream_t s = device ? stream : nullptr;
  const size_t units = core.batch * core.heads, D = core.head_dim;
  const uint64_t new_len = se->len + seq_len;
  if (new_len > se->cap) {
    const uint64_t cap = std::max<uint64_t>(new_len, std::max<uint64_t>(2 * se->cap, 16));
    DevBuf nk, nv;
    KIVI_TRY(nk.alloc_zero(units * cap * D * 4, s, "session suffix"));
    KIVI_TRY(nv.alloc_zero(units * cap * D * 4, s, "session suffix"));
    if (se->len > 0) {
      HIP_TRY(copy_units(nk.p, cap * D * 4, se->keys.p, se->cap * D * 4, se->len * D * 4, units, s), "suffix grow");
      HIP_TRY(copy_units(nv.p, cap * D * 4, se->values.p, se->cap * D * 4, se->len * D * 4, units, s), "suffix grow");
    }
    HIP_TRY(hipStreamSynchronize(s), "suffix grow");
    std::swap(se->keys.p, nk.p);
    std::swap(se->keys.bytes, nk.bytes);
    std::swap(se->values.p, nv.p);
    std::swap(se->values.bytes, nv.bytes);
    se->cap = cap;
  }
  const hipMemcpyKind kind = device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice;
  const size_t row = seq_len * D * 4;
  HIP_TRY(hipMemcpy2DAsync(se->keys.as<float>() + se->len * D, se->cap * D * 4, keys, row, row,
                           units, kind, s), "suffix append");
  HIP_TRY(hipMemcpy2DAsync(se->values.as<float>() + se->len * D, se->cap * D * 4, values, row, row,
                           units, kind, s), "suffix append");
  se->len = new_len;
  if (!device) return sync(s, "session append");
  return Status{};
}

Status batched_sessions(const kivi_session* const* sessions, size_t n, const float* queries,
                        size_t queries_len, size_t num_q_heads, float scale, float* out,
                        size_t out_len, bool device, hipStream_t stream) {
  KIVI_TRY(need_slice(sessions, n, "sessions"));
  if (n == 0) {
    if (queries_len != 0) return Err(KIVI_ERR_SHAPE, 0, queries_len);
    if (out_len != 0) return Err(KIVI_ERR_SHAPE, 0, out_len);
    return Status{};
  }
  for (size_t i = 0; i < n; ++i) KIVI_TRY(need(sessions[i], "sessions[i]"));
  const kivi_prefix_state* st = sessions[0]->prefix->state.get();
  for (size_t i = 1; i < n; ++i)
    if (sessions[i]->prefix->state.get() != st) return Err(KIVI_ERR_MISMATCHED_PREFIX, i, 0);
  const CacheCore& core = st->core;
  if (num_q_heads == 0 || num_q_heads % core.heads != 0)
    return Err(KIVI_ERR_QUERY_HEADS, num_q_heads, core.heads);
  size_t per, all;
  KIVI_TRY(mul4(core.batch, num_q_heads, core.head_dim, 1, &per));
  KIVI_TRY(mul(per, n, &all));
  if (queries_len != all) return Err(KIVI_ERR_SHAPE, all, queries_len);
  if (out_len != all) return Err(KIVI_ERR_SHAPE, all, out_len);
  KIVI_TRY(need_slice(queries, queries_len, "queries"));
  KIVI_TRY(need_slice(out, out_len, "out"));
  DeviceScope scope(core.device);
  hipStream_t s = device ? stream : nullptr;
  const float* dq = queries;
  float* dout = out;
  Scratch sq, so;
  if (!device) {
    KIVI_TRY(sq.get(all * 4, s, "sessions staging"));
    KIVI_TRY(so.get(all * 4, s, "sessions staging"));
    HIP_TRY(hipMemcpyAsync(sq.p, queries, all * 4, hipMemcpyHostToDevice, s), "sessions H2D");
    dq = sq.as<float>();
    dout = so.as<float>();
  }
  // One launch over the shared prefix per group of sessions when the packed-chunk path applies.
  std::vector<SessionDesc> descs(n);
  for (size_t i = 0; i < n; ++i) {
    const kivi_session* se = sessions[i];
    descs[i] = SessionDesc{se->keys.as<float>(), se->values.as<float>(), se->len, se->cap * core.head_dim};
  }
  SessionsProblem sp{};
  sp.cache = core.view();
  sp.st = core.state();
  sp.seq = core.seq;
  sp.n = static_cast<uint32_t>(n);
  sp.sessions = descs.data();
  sp.queries = dq;
  sp.out = dout;
  sp.qh = static_cast<uint32_t>(num_q_heads);
  sp.heads = static_cast<uint32_t>(core.heads);
  sp.batch = static_cast<uint32_t>(core.batch);
  sp.scale = scale;
  const size_t gq = num_q_heads / core.heads;
  const size_t ws_floats = n <= UINT32_MAX ? sessions_workspace_floats(sp) : 0;
  if (ws_floats > 0 && gq * core.head_dim <= kMaxGqD) {
    AttnSync& sync_ = st->batch;
    std::lock_guard<std::mutex> lock(sync_.mu);
    KIVI_TRY(sync_.reserve(ws_floats * sizeof(float)));
    KIVI_TRY(sync_.before(s));
    HIP_TRY(launch_sessions_attention(sp, sync_.workspace.as<float>(), s), "sessions attention");
    KIVI_TRY(sync_.after(s));
  } else {
    for (size_t i = 0; i < n; ++i) {
      kivi_session* se = const_cast<kivi_session*>(sessions[i]);  // its workspace only
      KIVI_TRY(attend(core, se->attn, se->keys.as<float>(), se->values.as<float>(), se->len,
                      se->cap * core.head_dim, dq + i * per, num_q_heads, scale, dout + i * per, s));
    }
  }
  if (!device) {
    HIP_TRY(hipMemcpyAsync(out, dout, all * 4, hipMemcpyDeviceToHost, s), "sessions D2H");
    return sync(s, "sessions attention");
  }
  return Status{};
}

// check_quant_args (src/quant.rs:235-273).
Status check_quant_args(size_t data_len, size_t batch, size_t heads, size_t tokens,
                        size_t head_dim, uint8_t bits, size_t group_size, bool per_channel) {
  KIVI_TRY(check_bits_group(bits, group_size));
  if (batch == 0) return Err(KIVI_ERR_ZERO_DIMENSION, 0, 0, "batch");
  if (heads == 0) return Err(KIVI_ERR_ZERO_DIMENSION, 0, 0, "heads");
  if (head_dim == 0) return Err(KIVI_ERR_ZERO_DIMENSION, 0, 0, "head_dim");
  if (per_channel) {
    if (tokens == 0 || tokens % group_size != 0) return Err(KIVI_ERR_TOKEN_GROUP, tokens, group_size);
  } else if (head_dim % group_size != 0) {
    return Err(KIVI_ERR_HEAD_DIM, head_dim, group_size);
  }
  size_t expected;
  KIVI_TRY(mul4(batch, heads, tokens, head_dim, &expected));
  if (data_len != expected) return Err(KIVI_ERR_SHAPE, expected, data_len);
  return Status{};
}

Status quantize(const float* data, size_t data_len, size_t batch, size_t heads, size_t tokens,
                size_t head_dim, uint8_t bits, size_t group_size, bool per_channel, bool device,
                hipStream_t stream, kivi_quantized** out) {
  KIVI_TRY(check_quant_args(data_len, batch, heads, tokens, head_dim, bits, group_size, per_channel));
  KIVI_TRY(need(out, "out"));
  KIVI_TRY(need_slice(data, data_len, "data"));
  if (head_dim > kMaxHeadDim) return Err(KIVI_ERR_UNSUPPORTED, head_dim, kMaxHeadDim, "head_dim");
  if (per_channel && group_size * head_dim > kMaxKeyTile)
    return Err(KIVI_ERR_UNSUPPORTED, group_size * head_dim, kMaxKeyTile, "group_size*head_dim");
  if (batch * heads > kMaxUnits) return Err(KIVI_ERR_UNSUPPORTED, batch * heads, kMaxUnits, "batch*heads");
  int dev = 0;
  KIVI_TRY(current_device(&dev));
  auto q = std::make_unique<kivi_quantized>();
  q->device = dev;
  q->axis = per_channel ? KIVI_AXIS_PER_CHANNEL : KIVI_AXIS_PER_TOKEN;
  q->bits = bits;
  q->group_size = group_size;
  q->batch = batch;
  q->heads = heads;
  q->tokens = tokens;
  q->head_dim = head_dim;
  const size_t units = batch * heads;
  q->n_codes = units * tokens * head_dim / (32 / bits);
  q->n_params = per_channel ? units * (tokens / group_size) * head_dim * 2
                            : units * tokens * (head_dim / group_size) * 2;
  hipStream_t s = device ? stream : nullptr;
  KIVI_TRY(q->codes.alloc_zero(q->n_codes * 4, s, "quantized codes"));
  KIVI_TRY(q->params.alloc_zero(q->n_params * 4, s, "quantized params"));
  const float* src = data;
  Scratch staging;
  if (!device) {
    KIVI_TRY(staging.get(data_len * 4, s, "quantize staging"));
    HIP_TRY(hipMemcpyAsync(staging.p, data, data_len * 4, hipMemcpyHostToDevice, s), "quantize H2D");
    src = staging.as<float>();
  }
  if (per_channel) {
    HIP_TRY(launch_quant_ref_keys(src, static_cast<uint32_t>(units), tokens, static_cast<uint32_t>(head_dim),
                                  bits, static_cast<uint32_t>(group_size), q->codes.as<uint32_t>(),
                                  q->params.as<float>(), s), "quantize_per_channel");
  } else {
    HIP_TRY(launch_quant_ref_values(src, static_cast<uint32_t>(units), tokens, static_cast<uint32_t>(head_dim),
                                    bits, static_cast<uint32_t>(group_size), q->codes.as<uint32_t>(),
                                    q->params.as<float>(), s), "quantize_per_token");
  }
  if (!device) KIVI_TRY(sync(s, "quantize"));
  *out = q.release();
  return Status{};
}

// With `device` the output is a device buffer written on `stream` (no staging, no sync).
Status quantized_read(const kivi_quantized* q, void* out, size_t out_len, size_t want,
                      int what /*0 codes 1 pytorch 2 params 3 dequant*/, bool device = false,
                      hipStream_t stream = nullptr) {
  KIVI_TRY(need(q, "quantized"));
  if (out_len != want) return Err(KIVI_ERR_SHAPE, want, out_len);
  if (want == 0) return Status{};
  KIVI_TRY(need(out, "out"));
  DeviceScope scope(q->device);
  hipStream_t s = device ? stream : nullptr;
  const uint32_t units = static_cast<uint32_t>(q->batch * q->heads);
  if (what == 0 || what == 2) {
    const void* src = what == 0 ? q->codes.p : q->params.p;
    HIP_TRY(hipMemcpyAsync(out, src, want * 4, device ? hipMemcpyDeviceToDevice : hipMemcpyDeviceToHost, s),
            "quantized read");
    return device ? Status{} : sync(s, "quantized read");
  }
  Scratch tmp;
  if (!device) KIVI_TRY(tmp.get(want * 4, s, "quantized read"));
  void* dst = device ? out : tmp.p;
  if (what == 1) {
    HIP_TRY(launch_pytorch_order(q->codes.as<uint32_t>(), units, q->tokens, static_cast<uint32_t>(q->head_dim),
                                 q->bits, static_cast<uint32_t>(q->group_size),
                                 q->axis == KIVI_AXIS_PER_CHANNEL, static_cast<uint32_t*>(dst), s),
            "pytorch_codes");
  } else {
    HIP_TRY(launch_dequant_ref(q->codes.as<uint32_t>(), q->params.as<float>(), units, q->tokens,
                               static_cast<uint32_t>(q->head_dim), q->bits,
                               static_cast<uint32_t>(q->group_size), q->axis == KIVI_AXIS_PER_CHANNEL,
                               static_cast<float*>(dst), s), "dequantize");
  }
  if (device) return Status{};
  HIP_TRY(hipMemcpyAsync(out, tmp.p, want * 4, hipMemcpyDeviceToHost, s), "quantized D2H");
  return sync(s, "quantized read");
}

}  // namespace

// ---------------------------------------------------------------- QualityGuard

// QualityGuard (src/guard.rs:37-258): the resident cache plus the fp32 tape of every appended
// token, here on the device ([units][cap][D], grown by doubling) so the fp32 attention it is
// scored against runs on the attention kernels (tape rows as the suffix of an empty cache).
struct kivi_guard {
  kivi_cache* cache = nullptr;
  DevBuf tk, tv;
  size_t cap = 0, seq = 0;
  float threshold = 0.f;
  uint32_t policy = KIVI_POLICY_RAISE_BITS;
  uint8_t max_bits = 8;
  size_t max_residual = 0;
  AttnSync dense;  // split partials of the fp32 attention
  std::vector<kivi_flush_check> last;  // checks of the last append
  std::mutex mu;
};

namespace {

// next_bits / next_residual (src/guard.rs:261-289).
bool guard_next_bits(uint8_t current, uint8_t max_bits, uint8_t* next) {
  const uint8_t n = current == 2 ? 4 : current == 4 ? 8 : 0;
  if (n == 0 || n > max_bits) return false;
  *next = n;
  return true;
}
bool guard_next_residual(size_t current, size_t group, size_t max_residual, size_t* next) {
  if (current >= max_residual) return false;
  const size_t doubled = current > SIZE_MAX / 2 ? SIZE_MAX : current * 2;
  const size_t n = doubled <= max_residual ? doubled : max_residual;
  if (!(n > current && n % group == 0)) return false;
  *next = n;
  return true;
}

// cosine_sim (src/guard.rs:362-377), sequential f32 sums as the reference.
float guard_cosine(const std::vector<float>& a, const std::vector<float>& b) {
  float dot = 0.f, na = 0.f, nb = 0.f;
  for (size_t i = 0; i < a.size() && i < b.size(); ++i) {
    dot += a[i] * b[i];
    na += a[i] * a[i];
    nb += b[i] * b[i];
  }
  const float denom = std::sqrt(na) * std::sqrt(nb);
  return denom == 0.f ? 1.f : dot / denom;
}

// push_history (src/guard.rs:237-245): `n` tokens of [units][n][D] host rows onto the tape.
Status guard_push(kivi_guard* g, const float* keys, const float* values, size_t n, hipStream_t s) {
  const CacheCore& core = g->cache->core;
  const size_t units = core.units(), D = core.head_dim;
  if (g->seq + n > g->cap) {
    const size_t cap = std::max({g->cap * 2, g->seq + n, static_cast<size_t>(64)});
    DevBuf nk, nv;
    KIVI_TRY(nk.alloc_zero(units * cap * D * sizeof(float), s, "guard tape"));
    KIVI_TRY(nv.alloc_zero(units * cap * D * sizeof(float), s, "guard tape"));
    if (g->seq > 0) {
      HIP_TRY(copy_units(nk.p, cap * D * 4, g->tk.p, g->cap * D * 4, g->seq * D * 4,
                         static_cast<uint32_t>(units), s), "guard tape");
      HIP_TRY(copy_units(nv.p, cap * D * 4, g->tv.p, g->cap * D * 4, g->seq * D * 4,
                         static_cast<uint32_t>(units), s), "guard tape");
    }
    std::swap(g->tk.p, nk.p);
    std::swap(g->tk.bytes, nk.bytes);
    std::swap(g->tv.p, nv.p);
    std::swap(g->tv.bytes, nv.bytes);
    g->cap = cap;
  }
  HIP_TRY(hipMemcpy2DAsync(g->tk.as<float>() + g->seq * D, g->cap * D * 4, keys, n * D * 4, n * D * 4,
                           units, hipMemcpyHostToDevice, s), "guard tape");
  HIP_TRY(hipMemcpy2DAsync(g->tv.as<float>() + g->seq * D, g->cap * D * 4, values, n * D * 4,
                           n * D * 4, units, hipMemcpyHostToDevice, s), "guard tape");
  g->seq += n;
  return sync(s, "guard tape");
}

// QualityGuard::cosine (src/guard.rs:218-235): cache attention against fp32 attention over
// the tape, both on the device, compared on the host.
Status guard_cosine_of(kivi_guard* g, const float* query, size_t query_len, size_t qh, float scale,
                       float* cosine) {
  kivi_cache* c = g->cache;
  const CacheCore& core = c->core;
  hipStream_t s = core.stream;
  const size_t n = core.batch * qh * core.head_dim;
  Scratch dq, dgot, dexp;
  KIVI_TRY(dq.get(query_len * 4, s, "guard staging"));
  KIVI_TRY(dgot.get(n * 4, s, "guard staging"));
  KIVI_TRY(dexp.get(n * 4, s, "guard staging"));
  HIP_TRY(hipMemcpyAsync(dq.p, query, query_len * 4, hipMemcpyHostToDevice, s), "guard H2D");
  KIVI_TRY(attend(core, c->attn, nullptr, nullptr, 0, 0, dq.as<float>(), qh, scale,
                  dgot.as<float>(), s));
  KIVI_TRY(attend(core, g->dense, g->tk.as<float>(), g->tv.as<float>(), g->seq, g->cap * core.head_dim,
                  dq.as<float>(), qh, scale, dexp.as<float>(), s, true));
  std::vector<float> got(n), expect(n);
  HIP_TRY(hipMemcpyAsync(got.data(), dgot.p, n * 4, hipMemcpyDeviceToHost, s), "guard D2H");
  HIP_TRY(hipMemcpyAsync(expect.data(), dexp.p, n * 4, hipMemcpyDeviceToHost, s), "guard D2H");
  KIVI_TRY(sync(s, "guard attention"));
  *cosine = guard_cosine(got, expect);
  return Status{};
}

// QualityGuard::apply (src/guard.rs:195-216): a new cache of the upgraded config holding the
// whole tape.
Status guard_apply(kivi_guard* g, const kivi_quality_upgrade& up) {
  kivi_config cfg = g->cache->core.cfg;
  if (up.kind == 0) {
    cfg.bits = static_cast<uint8_t>(up.to);
  } else {
    cfg.residual_length = up.to;
  }
  KIVI_TRY(check_config(cfg));
  const CacheCore& old = g->cache->core;
  auto nc = std::make_unique<kivi_cache>();
  KIVI_TRY(create_cache(&cfg, old.batch, old.heads, old.head_dim, nc.get()));
  nc->core.stream = old.stream;
  if (g->seq > 0) {
    hipStream_t s = old.stream;
    const size_t units = old.units(), D = old.head_dim;
    Scratch k, v;
    KIVI_TRY(k.get(units * g->seq * D * 4, s, "guard rebuild"));
    KIVI_TRY(v.get(units * g->seq * D * 4, s, "guard rebuild"));
    HIP_TRY(copy_units(k.p, g->seq * D * 4, g->tk.p, g->cap * D * 4, g->seq * D * 4,
                       static_cast<uint32_t>(units), s), "guard rebuild");
    HIP_TRY(copy_units(v.p, g->seq * D * 4, g->tv.p, g->cap * D * 4, g->seq * D * 4,
                       static_cast<uint32_t>(units), s), "guard rebuild");
    KIVI_TRY(nc->core.append_rows(k.as<float>(), v.as<float>(), g->seq, s));
    KIVI_TRY(sync(s, "guard rebuild"));
  }
  kivi_cache* prev = g->cache;
  g->cache = nc.release();
  kivi_cache_free(prev);
  return Status{};
}

}  // namespace

// ================================================================= C ABI

extern "C" {

void kivi_config_default(kivi_config* out) {
  if (out == nullptr) return;
  out->bits = 2;
  out->group_size = 32;
  out->residual_length = 128;
}

kivi_status kivi_config_try_new(uint8_t bits, size_t group_size, size_t residual_length,
                                kivi_config* out, kivi_error* err) {
  return guarded(err, [&] {
    kivi_config c{bits, group_size, residual_length};
    KIVI_TRY(check_config(c));
    KIVI_TRY(need(out, "out"));
    *out = c;
    return Status{};
  });
}

size_t kivi_memory_compressed_bytes(const kivi_memory_report* r) { return r ? compressed_bytes(*r) : 0; }

double kivi_memory_compression_ratio_vs_fp16(const kivi_memory_report* r) {
  if (r == nullptr) return 1.0;
  const size_t c = compressed_bytes(*r);
  return c == 0 ? 1.0 : static_cast<double>(r->fp16_baseline_bytes) / static_cast<double>(c);
}

double kivi_footprint_savings_vs_fp16(const kivi_prefix_footprint* f) {
  if (f == nullptr || f->shared_total_bytes == 0) return 1.0;
  return static_cast<double>(f->fp16_all_users_bytes) / static_cast<double>(f->shared_total_bytes);
}

kivi_status kivi_cache_new(const kivi_config* config, size_t batch, size_t num_kv_heads,
                           size_t head_dim, kivi_cache** out, kivi_error* err) {
  return guarded(err, [&] {
    auto c = std::make_unique<kivi_cache>();
    KIVI_TRY(create_cache(config, batch, num_kv_heads, head_dim, c.get()));
    KIVI_TRY(need(out, "out"));
    *out = c.release();
    return Status{};
  });
}

void kivi_cache_free(kivi_cache* cache) {
  if (cache == nullptr) return;
  DeviceScope scope(cache->core.device);
  (void)cache->settle();
  (void)hipStreamSynchronize(cache->core.stream);
  (void)cache->attn.drain();
  delete cache;
}

kivi_status kivi_cache_set_stream(kivi_cache* cache, void* stream, kivi_error* err) {
  return guarded(err, [&] {
    KIVI_TRY(need(cache, "cache"));
    KIVI_TRY(cache->settle());
    std::lock_guard<std::mutex> lock(cache->mu);
    const hipStream_t next = static_cast<hipStream_t>(stream);
    if (next != cache->core.stream) {
      // `*_device` calls made on the previous stream are not recorded as pending (host-pointer
      // calls on it follow them in stream order): they end before the new stream is used
      DeviceScope scope(cache->core.device);
      hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
      HIP_TRY(hipStreamIsCapturing(cache->core.stream, &cs), "set stream");
      if (cs == hipStreamCaptureStatusNone) HIP_TRY(hipStreamSynchronize(cache->core.stream), "set stream");
    }
    cache->core.stream = next;
    return Status{};
  });
}

kivi_config kivi_cache_config(const kivi_cache* c) { return c->core.cfg; }
size_t kivi_cache_batch_size(const kivi_cache* c) { return c->core.batch; }
size_t kivi_cache_num_kv_heads(const kivi_cache* c) { return c->core.heads; }
size_t kivi_cache_head_dim(const kivi_cache* c) { return c->core.head_dim; }
size_t kivi_cache_sequence_length(const kivi_cache* c) { return c->core.seq; }
size_t kivi_cache_key_residual_len(const kivi_cache* c) { return c->core.kres_len; }
size_t kivi_cache_value_residual_len(const kivi_cache* c) { return c->core.vres_len; }
size_t kivi_cache_quantized_key_tokens(const kivi_cache* c) { return c->core.kq; }
size_t kivi_cache_quantized_value_tokens(const kivi_cache* c) { return c->core.vq; }
size_t kivi_cache_tokens_until_key_flush(const kivi_cache* c) {
  const size_t r = c->core.cfg.residual_length;
  return r > c->core.kres_len ? r - c->core.kres_len : 0;
}
size_t kivi_cache_value_residual_slots_remaining(const kivi_cache* c) {
  const size_t r = c->core.cfg.residual_length;
  return r > c->core.vres_len ? r - c->core.vres_len : 0;
}

kivi_status kivi_cache_append(kivi_cache* cache, const float* keys, size_t keys_len,
                              const float* values, size_t values_len, size_t seq_len,
                              kivi_error* err) {
  return guarded(err, [&] {
    if (cache != nullptr) KIVI_TRY(cache->settle());
    return cache_append(cache, keys, keys_len, values, values_len, seq_len, false, nullptr);
  });
}

kivi_status kivi_cache_append_device(kivi_cache* cache, const float* keys, size_t keys_len,
                                     const float* values, size_t values_len, size_t seq_len,
                                     void* stream, kivi_error* err) {
  return guarded(err, [&] {
    KIVI_TRY(cache_append(cache, keys, keys_len, values, values_len, seq_len, true,
                          static_cast<hipStream_t>(stream)));
    cache->note_device(static_cast<hipStream_t>(stream));
    return Status{};
  });
}

kivi_status kivi_cache_attention(const kivi_cache* cache, const float* query, size_t query_len,
                                 size_t num_q_heads, float scale, float* out, size_t out_len,
                                 kivi_error* err) {
  return guarded(err, [&] {
    if (cache != nullptr) KIVI_TRY(const_cast<kivi_cache*>(cache)->settle());
    return cache_attention(cache, query, query_len, num_q_heads, scale, out, out_len, false, nullptr);
  });
}

kivi_status kivi_cache_attention_device(const kivi_cache* cache, const float* query,
                                        size_t query_len, size_t num_q_heads, float scale,
                                        float* out, size_t out_len, void* stream,
                                        kivi_error* err) {
  return guarded(err, [&] {
    KIVI_TRY(cache_attention(cache, query, query_len, num_q_heads, scale, out, out_len, true,
                             static_cast<hipStream_t>(stream)));
    const_cast<kivi_cache*>(cache)->note_device(static_cast<hipStream_t>(stream));
    return Status{};
  });
}

kivi_status kivi_cache_attention_device_noalloc(const kivi_cache* cache, const float* query,
                                                size_t query_len, size_t num_q_heads, float scale,
                                                float* out, size_t out_len, void* stream,
                                                kivi_error* err) {
  return guarded(err, [&] {
    KIVI_TRY(cache_attention_noalloc(cache, query, query_len, num_q_heads, scale, out, out_len,
                                     static_cast<hipStream_t>(stream)));
    const_cast<kivi_cache*>(cache)->note_device(static_cast<hipStream_t>(stream));
    return Status{};
  });
}

kivi_status kivi_cache_dequantize(const kivi_cache* cache, float* keys, size_t keys_len,
                                  float* values, size_t values_len, kivi_error* err) {
  return guarded(err, [&] {
    if (cache != nullptr) KIVI_TRY(const_cast<kivi_cache*>(cache)->settle());
    return cache_dequantize(cache, keys, keys_len, values, values_len, false, nullptr);
  });
}
kivi_status kivi_cache_dequantize_device(const kivi_cache* cache, float* keys, size_t keys_len,
                                         float* values, size_t values_len, void* stream,
                                         kivi_error* err) {
  return guarded(err, [&] {
    KIVI_TRY(cache_dequantize(cache, keys, keys_len, values, values_len, true, static_cast<hipStream_t>(stream)));
    const_cast<kivi_cache*>(cache)->note_device(static_cast<hipStream_t>(stream));
    return Status{};
  });
}

kivi_memory_report kivi_cache_memory(const kivi_cache* cache) { return cache->core.memory(); }

kivi_status kivi_cache_export_streams(const kivi_cache* cache, uint32_t* key_codes,
                                      size_t key_codes_len, float* key_params,
                                      size_t key_params_len, uint32_t* value_codes,
                                      size_t value_codes_len, float* value_params,
                                      size_t value_params_len, kivi_error* err) {
  return guarded(err, [&] {
    if (cache != nullptr) KIVI_TRY(const_cast<kivi_cache*>(cache)->settle());
    return cache_export(cache, key_codes, key_codes_len, key_params, key_params_len, value_codes,
                        value_codes_len, value_params, value_params_len, false, nullptr);
  });
}
kivi_status kivi_cache_export_streams_device(const kivi_cache* cache, uint32_t* key_codes,
                                             size_t key_codes_len, float* key_params,
                                             size_t key_params_len, uint32_t* value_codes,
                                             size_t value_codes_len, float* value_params,
                                             size_t value_params_len, void* stream,
                                             kivi_error* err) {
  return guarded(err, [&] {
    KIVI_TRY(cache_export(cache, key_codes, key_codes_len, key_params, key_params_len, value_codes,
                          value_codes_len, value_params, value_params_len, true,
                          static_cast<hipStream_t>(stream)));
    const_cast<kivi_cache*>(cache)->note_device(static_cast<hipStream_t>(stream));
    return Status{};
  });
}

kivi_status kivi_cache_reserve(kivi_cache* cache, size_t tokens, kivi_error* err) {
  return guarded(err, [&] {
    KIVI_TRY(need(cache, "cache"));
    KIVI_TRY(cache->settle());
    std::lock_guard<std::mutex> lock(cache->mu);
    DeviceScope scope(cache->core.device);
    KIVI_TRY(cache->core.ensure_capacity(tokens, cache->core.stream));
    return sync(cache->core.stream, "reserve");
  });
}

size_t kivi_cache_device_bytes(const kivi_cache* cache) {
  return cache ? cache->core.device_bytes() : 0;
}

kivi_status kivi_plan_device_bytes(const kivi_config* config, size_t batch, size_t num_kv_heads,
                                   size_t head_dim, size_t tokens, size_t* out, kivi_error* err) {
  return guarded(err, [&] {
    KIVI_TRY(need(config, "config"));
    KIVI_TRY(check_config(*config));
    if (batch == 0) return Err(KIVI_ERR_ZERO_DIMENSION, 0, 0, "batch");
    if (num_kv_heads == 0) return Err(KIVI_ERR_ZERO_DIMENSION, 0, 0, "num_kv_heads");
    if (head_dim == 0 || head_dim % config->group_size != 0)
      return Err(KIVI_ERR_HEAD_DIM, head_dim, config->group_size);
    KIVI_TRY(check_limits(*config, batch, num_kv_heads, head_dim));
    KIVI_TRY(need(out, "out"));
    CacheCore core;
    core.cfg = *config;
    core.batch = batch;
    core.heads = num_kv_heads;
    core.head_dim = head_dim;
    core.set_geometry();
    if (tokens > 0) core.geo.cap = core.capacity_for(tokens);
    *out = core.device_bytes();
    return Status{};
  });
}

kivi_status kivi_cache_share_prefix(const kivi_cache* cache, kivi_prefix** out, kivi_error* err) {
  return guarded(err, [&] {
    KIVI_TRY(need(cache, "cache"));
    KIVI_TRY(need(out, "out"));
    KIVI_TRY(const_cast<kivi_cache*>(cache)->settle());
    DeviceScope scope(cache->core.device);
    auto st = std::make_shared<kivi_prefix_state>();
    KIVI_TRY(cache->core.copy_into(st->core, cache->core.stream));
    // the prefix's |x| maxima also bound its fp32 residual / window rows (batched attention
    // dequantizes those into range-scaled f16 operands)
    HIP_TRY(launch_raise_row_max(st->core.view(), st->core.kres_len, st->core.vres_len, st->core.vhead,
                                 cache->core.stream), "prefix row maxima");
    KIVI_TRY(st->batch.init());
    KIVI_TRY(sync(cache->core.stream, "share_prefix"));
    st->prefix_bytes = compressed_bytes(st->core.memory());
    auto p = std::make_unique<kivi_prefix>();
    p->state = std::move(st);
    *out = p.release();
    return Status{};
  });
}

kivi_prefix* kivi_prefix_retain(kivi_prefix* prefix) {
  if (prefix != nullptr) prefix->refs.fetch_add(1, std::memory_order_relaxed);
  return prefix;
}

void kivi_prefix_release(kivi_prefix* prefix) {
  if (prefix == nullptr) return;
  if (prefix->refs.fetch_sub(1, std::memory_order_acq_rel) == 1) {
    DeviceScope scope(prefix->state->core.device);
    (void)hipDeviceSynchronize();
    delete prefix;
  }
}

kivi_config kivi_prefix_config(const kivi_prefix* p) { return p->state->core.cfg; }
size_t kivi_prefix_batch_size(const kivi_prefix* p) { return p->state->core.batch; }
size_t kivi_prefix_num_kv_heads(const kivi_prefix* p) { return p->state->core.heads; }
size_t kivi_prefix_head_dim(const kivi_prefix* p) { return p->state->core.head_dim; }
size_t kivi_prefix_prefix_tokens(const kivi_prefix* p) { return p->state->core.seq; }
size_t kivi_prefix_prefix_bytes(const kivi_prefix* p) { return p->state->prefix_bytes; }
int kivi_prefix_shares_allocation_with(const kivi_prefix* a, const kivi_prefix* b) {
  return (a != nullptr && b != nullptr && a->state.get() == b->state.get()) ? 1 : 0;
}

// SharedPrefix::footprint (src/prefix.rs:136-152).
kivi_prefix_footprint kivi_prefix_footprint_of(const kivi_prefix* p, size_t sessions,
                                               size_t question_tokens) {
  const CacheCore& c = p->state->core;
  const size_t elements = c.batch * c.heads * c.head_dim;
  const size_t question_bytes = sessions * question_tokens * elements * 2 * 4;
  const size_t fp16_per_user = 2 * (c.seq + question_tokens) * elements * 2;
  kivi_prefix_footprint f{};
  f.prefix_tokens = c.seq;
  f.question_tokens = question_tokens;
  f.sessions = sessions;
  f.prefix_bytes = p->state->prefix_bytes;
  f.question_bytes = question_bytes;
  f.shared_total_bytes = p->state->prefix_bytes + question_bytes;
  f.fp16_per_user_bytes = fp16_per_user;
  f.fp16_all_users_bytes = sessions * fp16_per_user;
  return f;
}

kivi_status kivi_prefix_session(kivi_prefix* prefix, kivi_session** out, kivi_error* err) {
  return guarded(err, [&] {
    KIVI_TRY(need(prefix, "prefix"));
    KIVI_TRY(need(out, "out"));
    auto s = std::make_unique<kivi_session>();
    {
      DeviceScope scope(prefix->state->core.device);
      KIVI_TRY(s->attn.init());
      KIVI_TRY(sync(nullptr, "session init"));
    }
    s->prefix = kivi_prefix_retain(prefix);
    *out = s.release();
    return Status{};
  });
}

void kivi_session_free(kivi_session* s) {
  if (s == nullptr) return;
  kivi_prefix* p = s->prefix;
  {
    DeviceScope scope(p->state->core.device);
    (void)hipDeviceSynchronize();
    delete s;
  }
  kivi_prefix_release(p);
}

kivi_prefix* kivi_session_prefix(const kivi_session* s) { return s->prefix; }
size_t kivi_session_prefix_tokens(const kivi_session* s) { return s->prefix->state->core.seq; }
size_t kivi_session_question_tokens(const kivi_session* s) { return s->len; }
size_t kivi_session_sequence_length(const kivi_session* s) { return s->prefix->state->core.seq + s->len; }

kivi_status kivi_session_append(kivi_session* session, const float* keys, size_t keys_len,
                                const float* values, size_t values_len, size_t seq_len,
                                kivi_error* err) {
  return guarded(err, [&] {
    if (session != nullptr) KIVI_TRY(session->dev.settle(nullptr));
    return session_append(session, keys, keys_len, values, values_len, seq_len, false, nullptr);
  });
}

kivi_status kivi_session_append_device(kivi_session* session, const float* keys,
                                       size_t keys_len, const float* values, size_t values_len,
                                       size_t seq_len, void* stream, kivi_error* err) {
  return guarded(err, [&] {
    KIVI_TRY(session_append(session, keys, keys_len, values, values_len, seq_len, true,
                            static_cast<hipStream_t>(stream)));
    session->dev.note(static_cast<hipStream_t>(stream));
    return Status{};
  });
}

kivi_status kivi_session_attention(const kivi_session* session, const float* query,
                                   size_t query_len, size_t num_q_heads, float scale, float* out,
                                   size_t out_len, kivi_error* err) {
  return guarded(err, [&] {
    if (session != nullptr) KIVI_TRY(const_cast<kivi_session*>(session)->dev.settle(nullptr));
    return session_attend(session, query, query_len, num_q_heads, scale, out, out_len, false, nullptr);
  });
}

kivi_status kivi_sessions_attention_device(const kivi_session* const* sessions, size_t n,
                                           const float* queries, size_t queries_len,
                                           size_t num_q_heads, float scale, float* out,
                                           size_t out_len, void* stream, kivi_error* err) {
  return guarded(err, [&] {
    KIVI_TRY(batched_sessions(sessions, n, queries, queries_len, num_q_heads, scale, out, out_len,
                              true, static_cast<hipStream_t>(stream)));
    for (size_t i = 0; i < n; ++i) const_cast<kivi_session*>(sessions[i])->dev.note(static_cast<hipStream_t>(stream));
    return Status{};
  });
}

kivi_status kivi_sessions_attention(const kivi_session* const* sessions, size_t n,
                                    const float* queries, size_t queries_len,
                                    size_t num_q_heads, float scale, float* out, size_t out_len,
                                    kivi_error* err) {
  return guarded(err, [&] {
    if (sessions != nullptr)
      for (size_t i = 0; i < n; ++i)
        if (sessions[i] != nullptr) KIVI_TRY(const_cast<kivi_session*>(sessions[i])->dev.settle(nullptr));
    return batched_sessions(sessions, n, queries, queries_len, num_q_heads, scale, out, out_len,
                            false, nullptr);
  });
}

kivi_status kivi_runtime_new(const kivi_config* config, size_t batch, size_t num_kv_heads,
                             size_t head_dim, kivi_runtime** out, kivi_error* err) {
  return guarded(err, [&] {
    auto rt = std::make_unique<kivi_runtime>();
    KIVI_TRY(create_cache(config, batch, num_kv_heads, head_dim, &rt->cache));
    KIVI_TRY(need(out, "out"));
    *out = rt.release();
    return Status{};
  });
}

void kivi_runtime_free(kivi_runtime* rt) {
  if (rt == nullptr) return;
  DeviceScope scope(rt->cache.core.device);
  (void)rt->cache.settle();
  (void)hipStreamSynchronize(rt->cache.core.stream);
  (void)rt->cache.attn.drain();
  delete rt;
}

kivi_cache* kivi_runtime_cache(kivi_runtime* rt) { return rt ? &rt->cache : nullptr; }

kivi_status kivi_runtime_prefill(kivi_runtime* rt, const float* keys, size_t keys_len,
                                 const float* values, size_t values_len, size_t seq_len,
                                 kivi_error* err) {
  return kivi_cache_append(rt ? &rt->cache : nullptr, keys, keys_len, values, values_len, seq_len, err);
}

// RuntimeKv::decode (src/runtime.rs:46-56): append(key, value, 1), then attention.
kivi_status kivi_runtime_decode(kivi_runtime* rt, const float* key, size_t key_len,
                                const float* value, size_t value_len, const float* query,
                                size_t query_len, size_t num_q_heads, float scale, float* out,
                                size_t out_len, kivi_error* err) {
  kivi_status st = kivi_cache_append(rt ? &rt->cache : nullptr, key, key_len, value, value_len, 1, err);
  if (st != KIVI_OK) return st;
  return kivi_cache_attention(&rt->cache, query, query_len, num_q_heads, scale, out, out_len, err);
}

kivi_status kivi_runtime_decode_device(kivi_runtime* rt, const float* key, size_t key_len,
                                       const float* value, size_t value_len, const float* query,
                                       size_t query_len, size_t num_q_heads, float scale,
                                       float* out, size_t out_len, void* stream,
                                       kivi_error* err) {
  bool fused = false;
  const kivi_status fs = guarded(err, [&] {
    return decode_fused(rt ? &rt->cache : nullptr, key, key_len, value, value_len, query, query_len,
                        num_q_heads, scale, out, out_len, static_cast<hipStream_t>(stream), &fused);
  });
  if (fs == KIVI_OK && fused) rt->cache.note_device(static_cast<hipStream_t>(stream));
  if (fs != KIVI_OK || fused) return fs;
  kivi_status st = kivi_cache_append_device(rt ? &rt->cache : nullptr, key, key_len, value,
                                            value_len, 1, stream, err);
  if (st != KIVI_OK) return st;
  return kivi_cache_attention_device(&rt->cache, query, query_len, num_q_heads, scale, out,
                                     out_len, stream, err);
}

kivi_status kivi_guard_new(const kivi_config* config, size_t batch, size_t num_kv_heads,
                           size_t head_dim, float threshold, uint32_t policy, uint8_t max_bits,
                           size_t max_residual, kivi_guard** out, kivi_error* err) {
  return guarded(err, [&] {
    if (policy != KIVI_POLICY_RAISE_BITS && policy != KIVI_POLICY_LENGTHEN_RESIDUAL)
      return Err(KIVI_ERR_UNSUPPORTED, policy, 1, "policy");
    auto g = std::make_unique<kivi_guard>();
    auto c = std::make_unique<kivi_cache>();
    KIVI_TRY(create_cache(config, batch, num_kv_heads, head_dim, c.get()));
    KIVI_TRY(g->dense.init());
    KIVI_TRY(need(out, "out"));
    g->cache = c.release();
    g->threshold = threshold;
    g->policy = policy;
    g->max_bits = max_bits;
    g->max_residual = max_residual;
    *out = g.release();
    return Status{};
  });
}

void kivi_guard_free(kivi_guard* guard) {
  if (guard == nullptr) return;
  {
    DeviceScope scope(guard->cache->core.device);
    (void)hipStreamSynchronize(guard->cache->core.stream);
    (void)guard->dense.drain();
  }
  kivi_cache_free(guard->cache);
  delete guard;
}

kivi_config kivi_guard_config(const kivi_guard* g) { return g->cache->core.cfg; }
kivi_cache* kivi_guard_cache(kivi_guard* g) { return g ? g->cache : nullptr; }
uint32_t kivi_guard_policy(const kivi_guard* g) { return g->policy; }
size_t kivi_guard_sequence_length(const kivi_guard* g) { return g->seq; }

kivi_status kivi_guard_append(kivi_guard* guard, const float* keys, size_t keys_len,
                              const float* values, size_t values_len, size_t seq_len,
                              const float* query, size_t query_len, size_t num_q_heads,
                              float scale, kivi_flush_check* checks, size_t checks_cap,
                              size_t* num_checks, kivi_error* err) {
  return guarded(err, [&]() -> Status {
    KIVI_TRY(need(guard, "guard"));
    KIVI_TRY(guard->cache->settle());
    const CacheCore& core0 = guard->cache->core;
    const size_t batch = core0.batch, heads = core0.heads, D = core0.head_dim;
    size_t expected, query_elems;
    KIVI_TRY(mul4(batch, heads, seq_len, D, &expected));
    if (keys_len != expected) return Err(KIVI_ERR_SHAPE, expected, keys_len);
    if (values_len != expected) return Err(KIVI_ERR_SHAPE, expected, values_len);
    if (num_q_heads == 0 || num_q_heads % heads != 0)
      return Err(KIVI_ERR_QUERY_HEADS, num_q_heads, heads);
    KIVI_TRY(mul4(batch, num_q_heads, D, 1, &query_elems));
    if (query_len != query_elems) return Err(KIVI_ERR_SHAPE, query_elems, query_len);
    KIVI_TRY(need_slice(query, query_len, "query"));
    if (seq_len > 0) {
      KIVI_TRY(need_slice(keys, keys_len, "keys"));
      KIVI_TRY(need_slice(values, values_len, "values"));
    }
    if (checks_cap > 0) KIVI_TRY(need(checks, "checks"));
    KIVI_TRY(need(num_checks, "num_checks"));
    std::lock_guard<std::mutex> lock(guard->mu);
    DeviceScope scope(core0.device);
    guard->last.clear();
    const size_t units = batch * heads;
    std::vector<float> ks, vs;
    size_t offset = 0;
    while (offset < seq_len) {
      const size_t room = kivi_cache_tokens_until_key_flush(guard->cache);
      const size_t take = std::min(room, seq_len - offset);
      // slice_tokens (src/guard.rs:291-311): tokens [offset, offset + take) of every unit
      ks.resize(units * take * D);
      vs.resize(units * take * D);
      for (size_t u = 0; u < units; ++u) {
        std::memcpy(&ks[u * take * D], keys + (u * seq_len + offset) * D, take * D * 4);
        std::memcpy(&vs[u * take * D], values + (u * seq_len + offset) * D, take * D * 4);
      }
      KIVI_TRY(cache_append(guard->cache, ks.data(), ks.size(), vs.data(), vs.size(), take, false,
                            nullptr));
      KIVI_TRY(guard_push(guard, ks.data(), vs.data(), take, guard->cache->core.stream));
      if (guard->cache->core.kres_len == 0) {
        // QualityGuard::check (src/guard.rs:148-172)
        kivi_flush_check fc{};
        KIVI_TRY(guard_cosine_of(guard, query, query_len, num_q_heads, scale, &fc.cosine_before));
        fc.cosine = fc.cosine_before;
        while (fc.cosine < guard->threshold) {
          // QualityGuard::propose (src/guard.rs:174-193)
          const kivi_config cfg = guard->cache->core.cfg;
          kivi_quality_upgrade up{};
          if (guard->policy == KIVI_POLICY_RAISE_BITS) {
            uint8_t to;
            if (!guard_next_bits(cfg.bits, guard->max_bits, &to)) break;
            up = kivi_quality_upgrade{0, cfg.bits, to};
          } else {
            size_t to;
            if (!guard_next_residual(cfg.residual_length, cfg.group_size, guard->max_residual, &to))
              break;
            up = kivi_quality_upgrade{1, cfg.residual_length, to};
          }
          if (fc.num_upgrades == KIVI_MAX_UPGRADES)
            return Err(KIVI_ERR_CAPACITY, fc.num_upgrades + 1, KIVI_MAX_UPGRADES, "upgrades");
          KIVI_TRY(guard_apply(guard, up));
          fc.upgrades[fc.num_upgrades++] = up;
          KIVI_TRY(guard_cosine_of(guard, query, query_len, num_q_heads, scale, &fc.cosine));
        }
        fc.sequence_tokens = guard->seq;
        guard->last.push_back(fc);
      }
      offset += take;
    }
    *num_checks = guard->last.size();
    for (size_t i = 0; i < guard->last.size() && i < checks_cap; ++i) checks[i] = guard->last[i];
    return Status{};
  });
}

size_t kivi_guard_last_checks(const kivi_guard* guard, size_t first, kivi_flush_check* checks,
                              size_t cap) {
  if (guard == nullptr || checks == nullptr) return 0;
  std::lock_guard<std::mutex> lock(const_cast<kivi_guard*>(guard)->mu);
  size_t n = 0;
  for (size_t i = first; i < guard->last.size() && n < cap; ++i) checks[n++] = guard->last[i];
  return n;
}

kivi_status kivi_quantize_per_channel(const float* data, size_t data_len, size_t batch,
                                      size_t heads, size_t tokens, size_t head_dim, uint8_t bits,
                                      size_t group_size, kivi_quantized** out, kivi_error* err) {
  return guarded(err, [&] {
    return quantize(data, data_len, batch, heads, tokens, head_dim, bits, group_size, true, false,
                    nullptr, out);
  });
}

kivi_status kivi_quantize_per_token(const float* data, size_t data_len, size_t batch,
                                    size_t heads, size_t tokens, size_t head_dim, uint8_t bits,
                                    size_t group_size, kivi_quantized** out, kivi_error* err) {
  return guarded(err, [&] {
    return quantize(data, data_len, batch, heads, tokens, head_dim, bits, group_size, false, false,
                    nullptr, out);
  });
}

kivi_status kivi_quantize_per_channel_device(const float* data, size_t data_len, size_t batch,
                                             size_t heads, size_t tokens, size_t head_dim,
                                             uint8_t bits, size_t group_size, void* stream,
                                             kivi_quantized** out, kivi_error* err) {
  return guarded(err, [&] {
    KIVI_TRY(quantize(data, data_len, batch, heads, tokens, head_dim, bits, group_size, true, true,
                      static_cast<hipStream_t>(stream), out));
    (*out)->dev.note(static_cast<hipStream_t>(stream));
    return Status{};
  });
}

kivi_status kivi_quantize_per_token_device(const float* data, size_t data_len, size_t batch,
                                           size_t heads, size_t tokens, size_t head_dim,
                                           uint8_t bits, size_t group_size, void* stream,
                                           kivi_quantized** out, kivi_error* err) {
  return guarded(err, [&] {
    KIVI_TRY(quantize(data, data_len, batch, heads, tokens, head_dim, bits, group_size, false, true,
                      static_cast<hipStream_t>(stream), out));
    (*out)->dev.note(static_cast<hipStream_t>(stream));
    return Status{};
  });
}

void kivi_quantized_free(kivi_quantized* q) {
  if (q == nullptr) return;
  DeviceScope scope(q->device);
  (void)hipDeviceSynchronize();
  delete q;
}

int kivi_quantized_axis(const kivi_quantized* q) { return q->axis; }
uint8_t kivi_quantized_bits(const kivi_quantized* q) { return q->bits; }
size_t kivi_quantized_group_size(const kivi_quantized* q) { return q->group_size; }
size_t kivi_quantized_num_tokens(const kivi_quantized* q) { return q->tokens; }
size_t kivi_quantized_code_bytes(const kivi_quantized* q) { return q->n_codes * 4; }
size_t kivi_quantized_metadata_bytes(const kivi_quantized* q) { return q->n_params * 4; }

kivi_status kivi_quantized_codes(const kivi_quantized* q, uint32_t* out, size_t out_len,
                                 kivi_error* err) {
  return guarded(err, [&] {
    if (q != nullptr) KIVI_TRY(q->dev.settle(nullptr));  // host reads use the default stream
    return quantized_read(q, out, out_len, q ? q->n_codes : 0, 0);
  });
}
kivi_status kivi_quantized_pytorch_codes(const kivi_quantized* q, uint32_t* out, size_t out_len,
                                         kivi_error* err) {
  return guarded(err, [&] {
    if (q != nullptr) KIVI_TRY(q->dev.settle(nullptr));  // host reads use the default stream
    return quantized_read(q, out, out_len, q ? q->n_codes : 0, 1);
  });
}
kivi_status kivi_quantized_scale_zero(const kivi_quantized* q, float* out, size_t out_len,
                                      kivi_error* err) {
  return guarded(err, [&] {
    if (q != nullptr) KIVI_TRY(q->dev.settle(nullptr));  // host reads use the default stream
    return quantized_read(q, out, out_len, q ? q->n_params : 0, 2);
  });
}
kivi_status kivi_quantized_dequantize(const kivi_quantized* q, float* out, size_t out_len,
                                      kivi_error* err) {
  return guarded(err, [&] {
    if (q != nullptr) KIVI_TRY(q->dev.settle(nullptr));  // host reads use the default stream
    const size_t n = q ? q->batch * q->heads * q->tokens * q->head_dim : 0;
    return quantized_read(q, out, out_len, n, 3);
  });
}
kivi_status kivi_quantized_pytorch_codes_device(const kivi_quantized* q, uint32_t* out,
                                                size_t out_len, void* stream, kivi_error* err) {
  return guarded(err, [&] {
    return quantized_read(q, out, out_len, q ? q->n_codes : 0, 1, true, static_cast<hipStream_t>(stream));
  });
}
kivi_status kivi_quantized_dequantize_device(const kivi_quantized* q, float* out, size_t out_len,
                                             void* stream, kivi_error* err) {
  return guarded(err, [&] {
    const size_t n = q ? q->batch * q->heads * q->tokens * q->head_dim : 0;
    return quantized_read(q, out, out_len, n, 3, true, static_cast<hipStream_t>(stream));
  });
}

const char* kivi_status_name(int32_t code) {
  switch (code) {
    case KIVI_OK: return "Ok";
    case KIVI_ERR_INVALID_BITS: return "InvalidBits";
    case KIVI_ERR_MISALIGNED_GROUP: return "MisalignedGroup";
    case KIVI_ERR_RESIDUAL_LENGTH: return "ResidualLength";
    case KIVI_ERR_HEAD_DIM: return "HeadDim";
    case KIVI_ERR_TOKEN_GROUP: return "TokenGroup";
    case KIVI_ERR_ZERO_DIMENSION: return "ZeroDimension";
    case KIVI_ERR_SHAPE: return "Shape";
    case KIVI_ERR_QUERY_HEADS: return "QueryHeads";
    case KIVI_ERR_EARLY_LAYERS: return "EarlyLayers";
    case KIVI_ERR_NULL_ARGUMENT: return "NullArgument";
    case KIVI_ERR_DEVICE: return "Device";
    case KIVI_ERR_CAPACITY: return "Capacity";
    case KIVI_ERR_UNSUPPORTED: return "Unsupported";
    case KIVI_ERR_MISMATCHED_PREFIX: return "MismatchedPrefix";
    default: return "Unknown";
  }
}

int32_t kivi_abi_version(void) { return KIVI_ABI_VERSION; }

int32_t kivi_device_count(void) { return device_count(); }

}  // extern "C"
