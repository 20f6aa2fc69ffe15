// kivi_oracle.cpp — TEST INFRASTRUCTURE ONLY.
//
// A CPU restatement of the reference crate bieli/kivi-cache-rs v0.6.0 (Rust, no
// dependencies), written in C++17 because the image has no Rust toolchain. It is the
// parity oracle for the HIP library and the "port" CPU baseline timed by bench.py.
// Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it,
// and only as the checker; nothing in the product links or calls it.
//
// Faithfulness rules (they make it bit-identical to the Rust build by construction):
//  * every loop runs in the reference's order; f32 arithmetic only; `mul_add` is
//    std::fma (libm fmaf, as Rust lowers it without target-cpu); `/` is IEEE division;
//    `f32::exp` is expf; the quantizers' `f32::min/max` are rust_min/rust_max below, the
//    compare-select x86-64 codegen of Rust's minnum/maxnum (NaN skipped, equal values keep
//    the running one, so a zero minimum keeps the sign of the group's first zero);
//  * built with -ffp-contract=off and without -ffast-math (oracle/Makefile);
//  * error checks in the reference's order, with the reference's Display text.
// Each function cites the reference lines it restates. The exported C API mirrors
// include/kivi.h under the prefix kivi_oracle_ so one binding drives both libraries.

#include "../include/kivi.h"

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <memory>
#include <new>
#include <vector>

namespace {

// f32::min / f32::max as the reference's x86-64 build runs them (src/quant.rs:303-304,
// 356-357). rustc lowers them to llvm.minnum / llvm.maxnum, and LLVM's x86 lowering of
// minnum(a, b) is minss(b, a) plus "a is NaN ? b : that": minss passes its second operand
// through on ties and NaNs, so minnum(a, b) = b < a ? b : a (a is never NaN here: it starts at
// +inf and only takes non-NaN values). glibc's fminf instead returns b on a tie of +0 and -0.
// The two differ only in the sign of a zero minimum; this is the reference's.
inline float rust_min(float acc, float x) { return x < acc ? x : acc; }
inline float rust_max(float acc, float x) { return x > acc ? x : acc; }

// ---------------------------------------------------------------- errors
// KiviError + Display (src/error.rs:5-95).

void set_error(kivi_error* e, int code, uint64_t a, uint64_t b, const char* name) {
  if (e == nullptr) return;
  std::memset(e, 0, sizeof(*e));
  e->code = code;
  e->a = a;
  e->b = b;
  if (name != nullptr) std::snprintf(e->name, sizeof(e->name), "%s", name);
  char* m = e->message;
  const size_t n = sizeof(e->message);
  const unsigned long long A = a, B = b;
  switch (code) {
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
      std::snprintf(m, n, "%s must be greater than zero", name ? name : "?");
      break;
    case KIVI_ERR_SHAPE:
      std::snprintf(m, n, "expected %llu elements, got %llu", A, B);
      break;
    case KIVI_ERR_QUERY_HEADS:
      std::snprintf(m, n, "num_q_heads %llu must be a positive multiple of num_kv_heads %llu", A, B);
      break;
    case KIVI_ERR_NULL_ARGUMENT:
      std::snprintf(m, n, "%s must not be null", name ? name : "?");
      break;
    default:
      std::snprintf(m, n, "error %d", code);
      break;
  }
}

struct Status {
  int code = KIVI_OK;
  uint64_t a = 0, b = 0;
  const char* name = nullptr;
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

kivi_status report(const Status& s, kivi_error* err) {
  if (s.ok()) {
    if (err != nullptr) std::memset(err, 0, sizeof(*err));
    return KIVI_OK;
  }
  set_error(err, s.code, s.a, s.b, s.name);
  return static_cast<kivi_status>(s.code);
}

// ---------------------------------------------------------------- config
// check_bits_group (src/config.rs:47-55), try_new (src/config.rs:31-45).

Status check_bits_group(uint8_t bits, size_t group_size) {
  if (!(bits == 2 || bits == 4 || bits == 8)) return Err(KIVI_ERR_INVALID_BITS, bits);
  if (group_size == 0 || (group_size * bits) % 32 != 0)
    return Err(KIVI_ERR_MISALIGNED_GROUP, group_size, bits);
  return Status{};
}

Status config_try_new(uint8_t bits, size_t group_size, size_t residual_length) {
  Status s = check_bits_group(bits, group_size);
  if (!s.ok()) return s;
  if (residual_length == 0 || residual_length % group_size != 0)
    return Err(KIVI_ERR_RESIDUAL_LENGTH, residual_length, group_size);
  return Status{};
}

// ---------------------------------------------------------------- quant
// PackedStream (src/quant.rs:37-44).
struct PackedStream {
  std::vector<uint32_t> codes;
  std::vector<float> params;  // interleaved [scale, zero], group-major
  size_t tokens = 0;
};

// scale_of (src/quant.rs:453-459).
float scale_of(float span, float levels) { return span == 0.0f ? 0.0f : span / levels; }

// round_half_even: floor-based, ties to even (src/quant.rs:475-485).
float round_half_even(float x) {
  const float fl = std::floor(x);
  const float frac = x - fl;
  if (frac > 0.5f) return fl + 1.0f;
  if (frac < 0.5f || static_cast<long long>(fl) % 2 == 0) return fl;
  return fl + 1.0f;
}

// quant_code (src/quant.rs:461-472).
uint32_t quant_code(float x, float zero, float scale, float levels) {
  if (scale == 0.0f) return 0;
  float rounded = round_half_even((x - zero) / scale);
  if (rounded < 0.0f) {
    rounded = 0.0f;
  } else if (rounded > levels) {
    rounded = levels;
  }
  return static_cast<uint32_t>(rounded);
}

// append_key_block: per-channel quantization over token groups (src/quant.rs:275-328).
void append_key_block(PackedStream& s, const float* data, size_t tokens, size_t head_dim,
                      uint8_t bits, size_t group_size) {
  if (tokens == 0) return;
  const float levels = static_cast<float>((1u << bits) - 1u);
  const size_t n_groups = tokens / group_size;
  const size_t ints_per_channel = group_size * bits / 32;
  s.codes.reserve(s.codes.size() + n_groups * head_dim * ints_per_channel);
  s.params.reserve(s.params.size() + n_groups * head_dim * 2);
  std::vector<float> mn(head_dim), mx(head_dim);
  for (size_t g = 0; g < n_groups; ++g) {
    std::fill(mn.begin(), mn.end(), INFINITY);
    std::fill(mx.begin(), mx.end(), -INFINITY);
    const size_t base = g * group_size * head_dim;
    for (size_t t = 0; t < group_size; ++t) {
      const float* row = data + base + t * head_dim;
      for (size_t d = 0; d < head_dim; ++d) {
        mn[d] = rust_min(mn[d], row[d]);
        mx[d] = rust_max(mx[d], row[d]);
      }
    }
    for (size_t d = 0; d < head_dim; ++d) {
      const float zero = mn[d];
      const float scale = scale_of(mx[d] - zero, levels);
      s.params.push_back(scale);
      s.params.push_back(zero);
      uint32_t word = 0, filled = 0;
      for (size_t t = 0; t < group_size; ++t) {
        const float x = data[base + t * head_dim + d];
        word |= quant_code(x, zero, scale, levels) << filled;
        filled += bits;
        if (filled == 32) {
          s.codes.push_back(word);
          word = 0;
          filled = 0;
        }
      }
    }
  }
  s.tokens += tokens;
}

// append_value_block: per-token quantization over channel groups (src/quant.rs:330-377).
void append_value_block(PackedStream& s, const float* data, size_t tokens, size_t head_dim,
                        uint8_t bits, size_t group_size) {
  if (tokens == 0) return;
  const float levels = static_cast<float>((1u << bits) - 1u);
  const size_t n_ch = head_dim / group_size;
  const size_t ints_per_group = group_size * bits / 32;
  s.codes.reserve(s.codes.size() + tokens * n_ch * ints_per_group);
  s.params.reserve(s.params.size() + tokens * n_ch * 2);
  for (size_t t = 0; t < tokens; ++t) {
    const float* row = data + t * head_dim;
    for (size_t cg = 0; cg < n_ch; ++cg) {
      const float* group = row + cg * group_size;
      float mn = INFINITY, mx = -INFINITY;
      for (size_t i = 0; i < group_size; ++i) {
        mn = rust_min(mn, group[i]);
        mx = rust_max(mx, group[i]);
      }
      const float scale = scale_of(mx - mn, levels);
      s.params.push_back(scale);
      s.params.push_back(mn);
      uint32_t word = 0, filled = 0;
      for (size_t i = 0; i < group_size; ++i) {
        word |= quant_code(group[i], mn, scale, levels) << filled;
        filled += bits;
        if (filled == 32) {
          s.codes.push_back(word);
          word = 0;
          filled = 0;
        }
      }
    }
  }
  s.tokens += tokens;
}

// dequant_keys (src/quant.rs:379-414).
void dequant_keys(const PackedStream& s, uint8_t bits, size_t group_size, size_t head_dim,
                  float* out) {
  if (s.tokens == 0) return;
  const size_t ints_per_channel = group_size * bits / 32;
  const uint32_t mask = (1u << bits) - 1u;
  const size_t n_groups = s.tokens / group_size;
  for (size_t g = 0; g < n_groups; ++g) {
    for (size_t d = 0; d < head_dim; ++d) {
      const size_t meta = 2 * (g * head_dim + d);
      const float scale = s.params[meta];
      const float zero = s.params[meta + 1];
      const size_t base = (g * head_dim + d) * ints_per_channel;
      size_t local = 0;
      for (size_t i = 0; i < ints_per_channel; ++i) {
        uint32_t word = s.codes[base + i];
        for (uint32_t left = 32; left > 0; left -= bits) {
          const float code = static_cast<float>(word & mask);
          const size_t t = g * group_size + local;
          out[t * head_dim + d] = std::fma(code, scale, zero);
          word >>= bits;
          ++local;
        }
      }
    }
  }
}

// dequant_values (src/quant.rs:416-451).
void dequant_values(const PackedStream& s, uint8_t bits, size_t group_size, size_t head_dim,
                    float* out) {
  if (s.tokens == 0) return;
  const size_t n_ch = head_dim / group_size;
  const size_t ints_per_group = group_size * bits / 32;
  const size_t ints_per_token = n_ch * ints_per_group;
  const uint32_t mask = (1u << bits) - 1u;
  for (size_t t = 0; t < s.tokens; ++t) {
    for (size_t cg = 0; cg < n_ch; ++cg) {
      const size_t meta = 2 * (t * n_ch + cg);
      const float scale = s.params[meta];
      const float zero = s.params[meta + 1];
      const size_t base = t * ints_per_token + cg * ints_per_group;
      size_t local = 0;
      for (size_t i = 0; i < ints_per_group; ++i) {
        uint32_t word = s.codes[base + i];
        for (uint32_t left = 32; left > 0; left -= bits) {
          const float code = static_cast<float>(word & mask);
          out[t * head_dim + cg * group_size + local] = std::fma(code, scale, zero);
          word >>= bits;
          ++local;
        }
      }
    }
  }
}

// check_quant_args (src/quant.rs:235-273).
Status check_quant_args(size_t data_len, size_t batch, size_t heads, size_t tokens,
                        size_t head_dim, uint8_t bits, size_t group_size, bool per_channel) {
  Status s = check_bits_group(bits, group_size);
  if (!s.ok()) return s;
  if (batch == 0) return Err(KIVI_ERR_ZERO_DIMENSION, 0, 0, "batch");
  if (heads == 0) return Err(KIVI_ERR_ZERO_DIMENSION, 0, 0, "heads");
  if (head_dim == 0) return Err(KIVI_ERR_ZERO_DIMENSION, 0, 0, "head_dim");
  if (per_channel) {
    if (tokens == 0 || tokens % group_size != 0)
      return Err(KIVI_ERR_TOKEN_GROUP, tokens, group_size);
  } else if (head_dim % group_size != 0) {
    return Err(KIVI_ERR_HEAD_DIM, head_dim, group_size);
  }
  const size_t expected = batch * heads * tokens * head_dim;
  if (data_len != expected) return Err(KIVI_ERR_SHAPE, expected, data_len);
  return Status{};
}

// ---------------------------------------------------------------- attention
// HeadView (src/attention.rs:9-16).
struct HeadView {
  const PackedStream* keys;
  const PackedStream* values;
  const float* key_residual;
  const float* value_residual;
  size_t key_res_len;
  size_t value_res_len;
};

// add16 / acc16 (src/attention.rs:271-287).
inline void add16(uint32_t word, float scale, float zero, float q, float* logits) {
  for (int slot = 0; slot < 16; ++slot) {
    const float recon = std::fma(static_cast<float>(word & 3u), scale, zero);
    logits[slot] = std::fma(recon, q, logits[slot]);
    word >>= 2;
  }
}
inline void acc16(uint32_t word, float scale, float zero, float w, float* out) {
  for (int slot = 0; slot < 16; ++slot) {
    const float recon = std::fma(static_cast<float>(word & 3u), scale, zero);
    out[slot] = std::fma(recon, w, out[slot]);
    word >>= 2;
  }
}

// key_logits_generic (src/attention.rs:143-177).
void key_logits_generic(const PackedStream& s, uint8_t bits, size_t group_size, size_t head_dim,
                        const float* query, float* logits) {
  const size_t ints_per_channel = group_size * bits / 32;
  const uint32_t mask = (1u << bits) - 1u;
  const size_t n_groups = s.tokens / group_size;
  for (size_t g = 0; g < n_groups; ++g) {
    float* lg = logits + g * group_size;
    std::fill(lg, lg + group_size, 0.0f);
    for (size_t d = 0; d < head_dim; ++d) {
      const float q = query[d];
      const size_t meta = 2 * (g * head_dim + d);
      const float scale = s.params[meta];
      const float zero = s.params[meta + 1];
      const size_t base = (g * head_dim + d) * ints_per_channel;
      size_t local = 0;
      for (size_t i = 0; i < ints_per_channel; ++i) {
        uint32_t word = s.codes[base + i];
        for (uint32_t left = 32; left > 0; left -= bits) {
          const float recon = std::fma(static_cast<float>(word & mask), scale, zero);
          lg[local] = std::fma(recon, q, lg[local]);
          word >>= bits;
          ++local;
        }
      }
    }
  }
}

// key_logits_2bit_g32 (src/attention.rs:179-200).
void key_logits_2bit_g32(const PackedStream& s, size_t head_dim, const float* query,
                         float* logits) {
  const size_t n_groups = s.tokens / 32;
  for (size_t g = 0; g < n_groups; ++g) {
    float* lg = logits + g * 32;
    std::fill(lg, lg + 32, 0.0f);
    for (size_t d = 0; d < head_dim; ++d) {
      const float q = query[d];
      const size_t meta = 2 * (g * head_dim + d);
      const float scale = s.params[meta];
      const float zero = s.params[meta + 1];
      const size_t base = (g * head_dim + d) * 2;
      add16(s.codes[base], scale, zero, q, lg);
      add16(s.codes[base + 1], scale, zero, q, lg + 16);
    }
  }
}

// key_logits dispatch (src/attention.rs:107-123).
void key_logits(const PackedStream& s, uint8_t bits, size_t group_size, size_t head_dim,
                const float* query, float* logits) {
  if (s.tokens == 0) return;
  if (bits == 2 && group_size == 32) {
    key_logits_2bit_g32(s, head_dim, query, logits);
  } else {
    key_logits_generic(s, bits, group_size, head_dim, query, logits);
  }
}

// value_mix_generic (src/attention.rs:202-239).
void value_mix_generic(const PackedStream& s, uint8_t bits, size_t group_size, size_t head_dim,
                       const float* weights, float* out) {
  const size_t n_ch = head_dim / group_size;
  const size_t ints_per_group = group_size * bits / 32;
  const size_t ints_per_token = n_ch * ints_per_group;
  const uint32_t mask = (1u << bits) - 1u;
  for (size_t t = 0; t < s.tokens; ++t) {
    const float w = weights[t];
    if (w == 0.0f) continue;
    for (size_t cg = 0; cg < n_ch; ++cg) {
      const size_t meta = 2 * (t * n_ch + cg);
      const float scale = s.params[meta];
      const float zero = s.params[meta + 1];
      const size_t base = t * ints_per_token + cg * ints_per_group;
      size_t local = 0;
      for (size_t i = 0; i < ints_per_group; ++i) {
        uint32_t word = s.codes[base + i];
        for (uint32_t left = 32; left > 0; left -= bits) {
          const float recon = std::fma(static_cast<float>(word & mask), scale, zero);
          const size_t d = cg * group_size + local;
          out[d] = std::fma(recon, w, out[d]);
          word >>= bits;
          ++local;
        }
      }
    }
  }
}

// value_mix_2bit_g32 (src/attention.rs:241-269).
void value_mix_2bit_g32(const PackedStream& s, size_t head_dim, const float* weights, float* out) {
  const size_t n_ch = head_dim / 32;
  for (size_t t = 0; t < s.tokens; ++t) {
    const float w = weights[t];
    if (w == 0.0f) continue;
    for (size_t cg = 0; cg < n_ch; ++cg) {
      const size_t meta = 2 * (t * n_ch + cg);
      const float scale = s.params[meta];
      const float zero = s.params[meta + 1];
      const size_t base = (t * n_ch + cg) * 2;
      acc16(s.codes[base], scale, zero, w, out + cg * 32);
      acc16(s.codes[base + 1], scale, zero, w, out + cg * 32 + 16);
    }
  }
}

// value_mix dispatch (src/attention.rs:125-141).
void value_mix(const PackedStream& s, uint8_t bits, size_t group_size, size_t head_dim,
               const float* weights, float* out) {
  if (s.tokens == 0) return;
  if (bits == 2 && group_size == 32) {
    value_mix_2bit_g32(s, head_dim, weights, out);
  } else {
    value_mix_generic(s, bits, group_size, head_dim, weights, out);
  }
}

// dense_logits (src/attention.rs:289-300).
void dense_logits(const float* rows, size_t n_tokens, size_t dim, const float* query,
                  float* logits) {
  for (size_t t = 0; t < n_tokens; ++t) {
    const float* row = rows + t * dim;
    float dot = 0.0f;
    for (size_t d = 0; d < dim; ++d) dot = std::fma(query[d], row[d], dot);
    logits[t] = dot;
  }
}

// dense_mix (src/attention.rs:302-315).
void dense_mix(const float* rows, size_t n_tokens, size_t dim, const float* weights, float* out) {
  for (size_t t = 0; t < n_tokens; ++t) {
    const float w = weights[t];
    if (w == 0.0f) continue;
    const float* row = rows + t * dim;
    for (size_t d = 0; d < dim; ++d) out[d] = std::fma(row[d], w, out[d]);
  }
}

// softmax: max, exp(x - max) with a sequential sum, multiply by 1/sum (src/attention.rs:317-333).
void softmax(float* xs, size_t n) {
  float max = -INFINITY;
  for (size_t i = 0; i < n; ++i)
    if (xs[i] > max) max = xs[i];
  float sum = 0.0f;
  for (size_t i = 0; i < n; ++i) {
    xs[i] = std::exp(xs[i] - max);
    sum += xs[i];
  }
  const float inv = 1.0f / sum;
  for (size_t i = 0; i < n; ++i) xs[i] *= inv;
}

// attend_head_with_suffix (src/attention.rs:47-105); attend_head is the empty-suffix case
// (src/attention.rs:18-41).
void attend_head_with_suffix(const HeadView& head, const float* suffix_keys,
                             const float* suffix_values, size_t suffix_len, const float* query,
                             uint8_t bits, size_t group_size, size_t head_dim, float scale,
                             float* logits, size_t logits_len, float* out) {
  const size_t kq = head.keys->tokens;
  const size_t prefix = kq + head.key_res_len;
  key_logits(*head.keys, bits, group_size, head_dim, query, logits);
  dense_logits(head.key_residual, head.key_res_len, head_dim, query, logits + kq);
  dense_logits(suffix_keys, suffix_len, head_dim, query, logits + prefix);
  for (size_t i = 0; i < logits_len; ++i) logits[i] *= scale;
  softmax(logits, logits_len);
  std::fill(out, out + head_dim, 0.0f);
  const size_t vq = head.values->tokens;
  value_mix(*head.values, bits, group_size, head_dim, logits, out);
  dense_mix(head.value_residual, head.value_res_len, head_dim, logits + vq, out);
  dense_mix(suffix_values, suffix_len, head_dim, logits + prefix, out);
}

// ---------------------------------------------------------------- cache
struct Cache;
struct PrefixState;

// copy_tokens (src/cache.rs:533-557).
void copy_tokens(float* dst, size_t dst_cap, size_t dst_off, const float* src, size_t src_seq,
                 size_t src_off, size_t count, size_t batch, size_t heads, size_t dim) {
  if (count == 0) return;
  for (size_t b = 0; b < batch; ++b)
    for (size_t h = 0; h < heads; ++h) {
      const size_t hi = b * heads + h;
      std::memcpy(dst + hi * dst_cap * dim + dst_off * dim, src + hi * src_seq * dim + src_off * dim,
                  count * dim * sizeof(float));
    }
}

// shift_residual (src/cache.rs:559-578).
void shift_residual(float* residual, size_t cap, size_t from, size_t keep, size_t batch,
                    size_t heads, size_t dim) {
  if (keep == 0 || from == 0) return;
  for (size_t b = 0; b < batch; ++b)
    for (size_t h = 0; h < heads; ++h) {
      float* base = residual + (b * heads + h) * cap * dim;
      std::memmove(base, base + from * dim, keep * dim * sizeof(float));
    }
}

// KiviCache (src/cache.rs:71-83).
struct Cache {
  kivi_config config{};
  size_t batch = 0, heads = 0, head_dim = 0;
  std::vector<PackedStream> key_streams, value_streams;
  std::vector<float> key_residual, value_residual;
  size_t key_res_len = 0, value_res_len = 0, seq_len = 0;

  size_t quantized_key_tokens() const { return key_streams.empty() ? 0 : key_streams[0].tokens; }
  size_t quantized_value_tokens() const {
    return value_streams.empty() ? 0 : value_streams[0].tokens;
  }

  // KiviCache::new (src/cache.rs:87-120).
  static Status create(const kivi_config& config, size_t batch, size_t num_kv_heads,
                       size_t head_dim, std::unique_ptr<Cache>* out) {
    if (batch == 0) return Err(KIVI_ERR_ZERO_DIMENSION, 0, 0, "batch");
    if (num_kv_heads == 0) return Err(KIVI_ERR_ZERO_DIMENSION, 0, 0, "num_kv_heads");
    if (head_dim == 0 || head_dim % config.group_size != 0)
      return Err(KIVI_ERR_HEAD_DIM, head_dim, config.group_size);
    auto c = std::make_unique<Cache>();
    c->config = config;
    c->batch = batch;
    c->heads = num_kv_heads;
    c->head_dim = head_dim;
    const size_t n = batch * num_kv_heads;
    c->key_streams.resize(n);
    c->value_streams.resize(n);
    c->key_residual.assign(n * config.residual_length * head_dim, 0.0f);
    c->value_residual.assign(n * config.residual_length * head_dim, 0.0f);
    *out = std::move(c);
    return Status{};
  }

  // KiviCache::append (src/cache.rs:186-214).
  Status append(const float* keys, size_t keys_len, const float* values, size_t values_len,
                size_t seq) {
    const size_t expected = batch * heads * seq * head_dim;
    if (keys_len != expected) return Err(KIVI_ERR_SHAPE, expected, keys_len);
    if (values_len != expected) return Err(KIVI_ERR_SHAPE, expected, values_len);
    append_keys(keys, seq);
    append_values(values, seq);
    seq_len += seq;
    return Status{};
  }

  // append_keys (src/cache.rs:382-405).
  void append_keys(const float* keys, size_t seq) {
    const size_t r = config.residual_length;
    size_t offset = 0;
    while (offset < seq) {
      const size_t space = r - key_res_len;
      const size_t take = space < seq - offset ? space : seq - offset;
      copy_tokens(key_residual.data(), r, key_res_len, keys, seq, offset, take, batch, heads,
                  head_dim);
      key_res_len += take;
      offset += take;
      if (key_res_len == r) flush_keys();
    }
  }

  // flush_keys (src/cache.rs:407-430).
  void flush_keys() {
    const size_t r = config.residual_length;
    for (size_t b = 0; b < batch; ++b)
      for (size_t h = 0; h < heads; ++h) {
        const size_t hi = b * heads + h;
        append_key_block(key_streams[hi], key_residual.data() + hi * r * head_dim, r, head_dim,
                         config.bits, config.group_size);
      }
    key_res_len = 0;
  }

  // append_values (src/cache.rs:432-484).
  void append_values(const float* values, size_t seq) {
    const size_t r = config.residual_length;
    if (seq >= r) {
      quantize_value_residual_prefix(value_res_len);
      const size_t quant_n = seq - r;
      if (quant_n > 0) quantize_value_input(values, seq, 0, quant_n);
      copy_tokens(value_residual.data(), r, 0, values, seq, quant_n, r, batch, heads, head_dim);
      value_res_len = r;
      return;
    }
    const size_t combined = value_res_len + seq;
    const size_t drop = combined > r ? combined - r : 0;
    if (drop > 0) {
      quantize_value_residual_prefix(drop);
      const size_t keep = value_res_len - drop;
      shift_residual(value_residual.data(), r, drop, keep, batch, heads, head_dim);
      value_res_len = keep;
    }
    copy_tokens(value_residual.data(), r, value_res_len, values, seq, 0, seq, batch, heads,
                head_dim);
    value_res_len += seq;
  }

  // quantize_value_residual_prefix (src/cache.rs:486-510).
  void quantize_value_residual_prefix(size_t n) {
    if (n == 0) return;
    const size_t cap = config.residual_length;
    for (size_t b = 0; b < batch; ++b)
      for (size_t h = 0; h < heads; ++h) {
        const size_t hi = b * heads + h;
        append_value_block(value_streams[hi], value_residual.data() + hi * cap * head_dim, n,
                           head_dim, config.bits, config.group_size);
      }
  }

  // quantize_value_input (src/cache.rs:512-530).
  void quantize_value_input(const float* values, size_t seq, size_t offset, size_t count) {
    for (size_t b = 0; b < batch; ++b)
      for (size_t h = 0; h < heads; ++h) {
        const size_t hi = b * heads + h;
        append_value_block(value_streams[hi], values + hi * seq * head_dim + offset * head_dim,
                           count, head_dim, config.bits, config.group_size);
      }
  }

  // KiviCache::attention (src/cache.rs:224-279).
  Status attention(const float* query, size_t query_len, size_t num_q_heads, float scale,
                   float* out) const {
    if (num_q_heads == 0 || num_q_heads % heads != 0)
      return Err(KIVI_ERR_QUERY_HEADS, num_q_heads, heads);
    const size_t expected = batch * num_q_heads * head_dim;
    if (query_len != expected) return Err(KIVI_ERR_SHAPE, expected, query_len);
    std::fill(out, out + expected, 0.0f);
    if (seq_len == 0) return Status{};
    std::vector<float> logits(seq_len, 0.0f);
    const size_t group = num_q_heads / heads;
    const size_t cap = config.residual_length;
    for (size_t b = 0; b < batch; ++b)
      for (size_t qh = 0; qh < num_q_heads; ++qh) {
        const size_t kvh = qh / group;
        const size_t hi = b * heads + kvh;
        const size_t slot = hi * cap * head_dim;
        HeadView view{&key_streams[hi], &value_streams[hi], key_residual.data() + slot,
                      value_residual.data() + slot, key_res_len, value_res_len};
        attend_head_with_suffix(view, nullptr, nullptr, 0,
                                query + (b * num_q_heads + qh) * head_dim, config.bits,
                                config.group_size, head_dim, scale, logits.data(), seq_len,
                                out + (b * num_q_heads + qh) * head_dim);
      }
    return Status{};
  }

  // KiviCache::dequantize (src/cache.rs:282-325).
  void dequantize(float* keys, float* values) const {
    const size_t n = batch * heads * seq_len * head_dim;
    std::fill(keys, keys + n, 0.0f);
    std::fill(values, values + n, 0.0f);
    const size_t kq = quantized_key_tokens();
    const size_t vq = quantized_value_tokens();
    const size_t cap = config.residual_length;
    for (size_t b = 0; b < batch; ++b)
      for (size_t h = 0; h < heads; ++h) {
        const size_t hi = b * heads + h;
        const size_t dst = hi * seq_len * head_dim;
        const size_t slot = hi * cap * head_dim;
        if (kq > 0)
          dequant_keys(key_streams[hi], config.bits, config.group_size, head_dim, keys + dst);
        if (key_res_len > 0)
          std::memcpy(keys + dst + kq * head_dim, key_residual.data() + slot,
                      key_res_len * head_dim * sizeof(float));
        if (vq > 0)
          dequant_values(value_streams[hi], config.bits, config.group_size, head_dim,
                         values + dst);
        if (value_res_len > 0)
          std::memcpy(values + dst + vq * head_dim, value_residual.data() + slot,
                      value_res_len * head_dim * sizeof(float));
      }
  }

  // KiviCache::memory (src/cache.rs:362-380).
  kivi_memory_report memory() const {
    kivi_memory_report r{};
    for (const auto& s : key_streams) {
      r.key_code_bytes += s.codes.size() * 4;
      r.key_metadata_bytes += s.params.size() * 4;
    }
    for (const auto& s : value_streams) {
      r.value_code_bytes += s.codes.size() * 4;
      r.value_metadata_bytes += s.params.size() * 4;
    }
    const size_t elements = batch * heads * head_dim;
    r.tokens = seq_len;
    r.key_residual_bytes = key_res_len * elements * 4;
    r.value_residual_bytes = value_res_len * elements * 4;
    r.residual_capacity_bytes = 2 * config.residual_length * elements * 4;
    r.fp16_baseline_bytes = 2 * seq_len * elements * 2;
    r.fp32_baseline_bytes = 2 * seq_len * elements * 4;
    return r;
  }
};

size_t compressed_bytes(const kivi_memory_report& r) {
  return r.key_code_bytes + r.key_metadata_bytes + r.value_code_bytes + r.value_metadata_bytes +
         r.key_residual_bytes + r.value_residual_bytes;
}

// ---------------------------------------------------------------- prefix
// PrefixState (src/prefix.rs:14-27): a deep copy of the cache plus its byte count.
struct PrefixState {
  Cache cache;
  size_t prefix_bytes = 0;
};

}  // namespace

// Opaque handles of the oracle's C API.
struct kivi_oracle_cache {
  std::unique_ptr<Cache> c;
};
struct kivi_oracle_prefix {
  std::shared_ptr<const PrefixState> state;  // SharedPrefix = Arc<PrefixState> (src/prefix.rs:33-35)
};
struct kivi_oracle_session {
  kivi_oracle_prefix prefix;  // RagSession (src/prefix.rs:41-46)
  std::vector<float> local_keys, local_values;
  size_t local_len = 0;
};
struct kivi_oracle_runtime {
  kivi_oracle_cache cache;
};
// QualityGuard (src/guard.rs:37-47).
struct kivi_oracle_guard {
  kivi_oracle_cache cache;  // the resident cache, replaced by a rebuild
  std::vector<float> keys, values;
  size_t seq = 0;
  float threshold = 0.f;
  uint8_t max_bits = 8;
  size_t max_residual = 0;
  uint32_t policy = KIVI_POLICY_RAISE_BITS;
  std::vector<kivi_flush_check> last;
};
struct kivi_oracle_quantized {
  std::vector<PackedStream> streams;  // QuantizedTensor (src/quant.rs:26-35)
  size_t batch = 0, heads = 0, head_dim = 0, tokens = 0;
  uint8_t bits = 0;
  size_t group_size = 0;
  int axis = 0;
};

namespace {

// splice_tokens (src/prefix.rs:292-318).
void splice_tokens(float* dst, const float* old, const float* fresh, size_t old_len,
                   size_t new_len, size_t batch, size_t heads, size_t dim) {
  const size_t total = old_len + new_len;
  for (size_t b = 0; b < batch; ++b)
    for (size_t h = 0; h < heads; ++h) {
      const size_t hi = b * heads + h;
      float* d = dst + hi * total * dim;
      if (old_len > 0) std::memcpy(d, old + hi * old_len * dim, old_len * dim * sizeof(float));
      std::memcpy(d + old_len * dim, fresh + hi * new_len * dim, new_len * dim * sizeof(float));
    }
}

// RagSession::attention (src/prefix.rs:228-289).
Status session_attention(const kivi_oracle_session& s, const float* query, size_t query_len,
                         size_t num_q_heads, float scale, float* out) {
  const Cache& st = s.prefix.state->cache;
  if (num_q_heads == 0 || num_q_heads % st.heads != 0)
    return Err(KIVI_ERR_QUERY_HEADS, num_q_heads, st.heads);
  const size_t expected = st.batch * num_q_heads * st.head_dim;
  if (query_len != expected) return Err(KIVI_ERR_SHAPE, expected, query_len);
  const size_t total = st.seq_len + s.local_len;
  std::fill(out, out + expected, 0.0f);
  if (total == 0) return Status{};
  std::vector<float> logits(total, 0.0f);
  const size_t group = num_q_heads / st.heads;
  const size_t cap = st.config.residual_length;
  const size_t dim = st.head_dim;
  for (size_t b = 0; b < st.batch; ++b)
    for (size_t qh = 0; qh < num_q_heads; ++qh) {
      const size_t kvh = qh / group;
      const size_t hi = b * st.heads + kvh;
      const size_t slot = hi * cap * dim;
      const size_t local = hi * s.local_len * dim;
      HeadView view{&st.key_streams[hi], &st.value_streams[hi], st.key_residual.data() + slot,
                    st.value_residual.data() + slot, st.key_res_len, st.value_res_len};
      attend_head_with_suffix(view, s.local_keys.data() + local, s.local_values.data() + local,
                              s.local_len, query + (b * num_q_heads + qh) * dim, st.config.bits,
                              st.config.group_size, dim, scale, logits.data(), total,
                              out + (b * num_q_heads + qh) * dim);
    }
  return Status{};
}

template <class F>
kivi_status guarded(kivi_error* err, F&& f) {
  try {
    return report(f(), err);
  } catch (const std::bad_alloc&) {
    return report(Err(KIVI_ERR_CAPACITY), err);
  }
}

Status need(const void* p, const char* name) {
  return p == nullptr ? Err(KIVI_ERR_NULL_ARGUMENT, 0, 0, name) : Status{};
}

// Pointers may be NULL only for empty slices (Rust's empty &[f32]).
Status need_slice(const void* p, size_t len, const char* name) {
  return (p == nullptr && len != 0) ? Err(KIVI_ERR_NULL_ARGUMENT, 0, 0, name) : Status{};
}

Status quantize_impl(const float* data, size_t data_len, size_t batch, size_t heads,
                     size_t tokens, size_t head_dim, uint8_t bits, size_t group_size,
                     bool per_channel, kivi_oracle_quantized** out) {
  Status s = check_quant_args(data_len, batch, heads, tokens, head_dim, bits, group_size,
                              per_channel);
  if (!s.ok()) return s;
  if (!(s = need(out, "out")).ok()) return s;
  if (!(s = need_slice(data, data_len, "data")).ok()) return s;
  auto q = std::make_unique<kivi_oracle_quantized>();
  q->streams.resize(batch * heads);
  for (size_t b = 0; b < batch; ++b)
    for (size_t h = 0; h < heads; ++h) {
      const size_t hi = b * heads + h;
      const float* src = data + hi * tokens * head_dim;
      if (per_channel)
        append_key_block(q->streams[hi], src, tokens, head_dim, bits, group_size);
      else
        append_value_block(q->streams[hi], src, tokens, head_dim, bits, group_size);
    }
  q->batch = batch;
  q->heads = heads;
  q->head_dim = head_dim;
  q->tokens = tokens;
  q->bits = bits;
  q->group_size = group_size;
  q->axis = per_channel ? KIVI_AXIS_PER_CHANNEL : KIVI_AXIS_PER_TOKEN;
  *out = q.release();
  return Status{};
}

}  // namespace

// ================================================================= C API (oracle)
// ---------------------------------------------------------------- QualityGuard helpers

// next_bits (src/guard.rs:261-272).
bool guard_next_bits(uint8_t current, uint8_t max_bits, uint8_t* next) {
  uint8_t n;
  switch (current) {
    case 2: n = 4; break;
    case 4: n = 8; break;
    default: return false;
  }
  if (n > max_bits) return false;
  *next = n;
  return true;
}

// next_residual (src/guard.rs:274-289).
bool guard_next_residual(size_t current, size_t group_size, size_t max_residual, size_t* next) {
  if (current >= max_residual) return false;
  const size_t doubled = current > SIZE_MAX / 2 ? SIZE_MAX : current * 2;  // saturating_mul
  const size_t n = doubled <= max_residual ? doubled : max_residual;
  if (n > current && n % group_size == 0) {
    *next = n;
    return true;
  }
  return false;
}

// slice_tokens (src/guard.rs:291-311).
std::vector<float> guard_slice(const float* src, size_t batch, size_t heads, size_t seq,
                               size_t start, size_t len, size_t dim) {
  std::vector<float> out(batch * heads * len * dim, 0.f);
  for (size_t b = 0; b < batch; ++b)
    for (size_t h = 0; h < heads; ++h) {
      const size_t hi = b * heads + h;
      std::memcpy(&out[hi * len * dim], src + hi * seq * dim + start * dim, len * dim * 4);
    }
  return out;
}

// concat_tokens (src/guard.rs:313-342).
std::vector<float> guard_concat(const std::vector<float>& old, const std::vector<float>& add,
                                size_t old_len, size_t new_len, size_t batch, size_t heads,
                                size_t dim) {
  const size_t total = old_len + new_len;
  std::vector<float> dst(batch * heads * total * dim, 0.f);
  for (size_t b = 0; b < batch; ++b)
    for (size_t h = 0; h < heads; ++h) {
      const size_t hi = b * heads + h;
      if (old_len > 0)
        std::memcpy(&dst[hi * total * dim], &old[hi * old_len * dim], old_len * dim * 4);
      std::memcpy(&dst[hi * total * dim + old_len * dim], &add[hi * new_len * dim], new_len * dim * 4);
    }
  return dst;
}

// fp32_attention (src/guard.rs:344-385): f32 sums in token and dim order, expf, maxNum fold.
std::vector<float> guard_fp32_attention(const float* query, const std::vector<float>& keys,
                                        const std::vector<float>& values, size_t batch,
                                        size_t kv_heads, size_t q_heads, size_t seq, size_t dim,
                                        float scale) {
  std::vector<float> out(batch * q_heads * dim, 0.f);
  const size_t group = q_heads / kv_heads;
  std::vector<float> logits(seq, 0.f);
  for (size_t b = 0; b < batch; ++b)
    for (size_t qh = 0; qh < q_heads; ++qh) {
      const size_t kvh = qh / group;
      const float* q = query + (b * q_heads + qh) * dim;
      const size_t base = (b * kv_heads + kvh) * seq * dim;
      for (size_t t = 0; t < seq; ++t) {
        float dot = 0.f;
        for (size_t d = 0; d < dim; ++d) dot += q[d] * keys[base + t * dim + d];
        logits[t] = dot * scale;
      }
      float mx = -INFINITY;
      for (float l : logits) mx = fmaxf(mx, l);
      float sum = 0.f;
      for (float& l : logits) {
        l = expf(l - mx);
        sum += l;
      }
      float* y = &out[(b * q_heads + qh) * dim];
      for (size_t d = 0; d < dim; ++d) y[d] = 0.f;
      for (size_t t = 0; t < seq; ++t) {
        const float w = logits[t] / sum;
        for (size_t d = 0; d < dim; ++d) y[d] += w * values[base + t * dim + d];
      }
    }
  return out;
}

// cosine_sim (src/guard.rs:387-402).
float guard_cosine_sim(const std::vector<float>& a, const std::vector<float>& b) {
  float dot = 0.f, na = 0.f, nb = 0.f;
  for (size_t i = 0; i < a.size() && i < b.size(); ++i) {
    dot += a[i] * b[i];
    na += a[i] * a[i];
    nb += b[i] * b[i];
  }
  const float denom = std::sqrt(na) * std::sqrt(nb);
  return denom == 0.f ? 1.f : dot / denom;
}

// QualityGuard::cosine (src/guard.rs:218-235).
Status guard_cosine(const kivi_oracle_guard& g, const float* query, size_t query_len,
                    size_t num_q_heads, float scale, float* cosine) {
  const Cache& c = *g.cache.c;
  std::vector<float> got(c.batch * num_q_heads * c.head_dim);
  Status s = c.attention(query, query_len, num_q_heads, scale, got.data());
  if (!s.ok()) return s;
  const std::vector<float> expect = guard_fp32_attention(
      query, g.keys, g.values, c.batch, c.heads, num_q_heads, g.seq, c.head_dim, scale);
  *cosine = guard_cosine_sim(got, expect);
  return Status{};
}

// QualityGuard::apply (src/guard.rs:195-216).
Status guard_apply(kivi_oracle_guard& g, const kivi_quality_upgrade& up) {
  const kivi_config cur = g.cache.c->config;
  kivi_config cfg{};
  Status s = up.kind == 0 ? config_try_new(static_cast<uint8_t>(up.to), cur.group_size, cur.residual_length)
                          : config_try_new(cur.bits, cur.group_size, up.to);
  if (!s.ok()) return s;
  cfg.bits = up.kind == 0 ? static_cast<uint8_t>(up.to) : cur.bits;
  cfg.group_size = cur.group_size;
  cfg.residual_length = up.kind == 0 ? cur.residual_length : up.to;
  std::unique_ptr<Cache> c;
  if (!(s = Cache::create(cfg, g.cache.c->batch, g.cache.c->heads, g.cache.c->head_dim, &c)).ok()) return s;
  if (g.seq > 0 &&
      !(s = c->append(g.keys.data(), g.keys.size(), g.values.data(), g.values.size(), g.seq)).ok())
    return s;
  g.cache.c = std::move(c);
  return Status{};
}

extern "C" {

void kivi_oracle_config_default(kivi_config* out) {
  if (out == nullptr) return;
  out->bits = 2;
  out->group_size = 32;
  out->residual_length = 128;
}

kivi_status kivi_oracle_config_try_new(uint8_t bits, size_t group_size, size_t residual_length,
                                       kivi_config* out, kivi_error* err) {
  return guarded(err, [&] {
    Status s = config_try_new(bits, group_size, residual_length);
    if (!s.ok()) return s;
    if (!(s = need(out, "out")).ok()) return s;
    out->bits = bits;
    out->group_size = group_size;
    out->residual_length = residual_length;
    return Status{};
  });
}

size_t kivi_oracle_memory_compressed_bytes(const kivi_memory_report* r) {
  return r ? compressed_bytes(*r) : 0;
}

// MemoryReport::compression_ratio_vs_fp16 (src/cache.rs:50-57).
double kivi_oracle_memory_compression_ratio_vs_fp16(const kivi_memory_report* r) {
  if (r == nullptr) return 1.0;
  const size_t c = compressed_bytes(*r);
  return c == 0 ? 1.0 : static_cast<double>(r->fp16_baseline_bytes) / static_cast<double>(c);
}

// SharedPrefixFootprint::savings_vs_fp16 (src/prefix.rs:62-71).
double kivi_oracle_footprint_savings_vs_fp16(const kivi_prefix_footprint* f) {
  if (f == nullptr || f->shared_total_bytes == 0) return 1.0;
  return static_cast<double>(f->fp16_all_users_bytes) / static_cast<double>(f->shared_total_bytes);
}

kivi_status kivi_oracle_cache_new(const kivi_config* config, size_t batch, size_t num_kv_heads,
                                  size_t head_dim, kivi_oracle_cache** out, kivi_error* err) {
  return guarded(err, [&] {
    Status s = need(config, "config");
    if (!s.ok()) return s;
    if (!(s = need(out, "out")).ok()) return s;
    // The C ABI validates the config first (see kivi.h); the reference's own checks follow.
    if (!(s = config_try_new(config->bits, config->group_size, config->residual_length)).ok())
      return s;
    std::unique_ptr<Cache> c;
    if (!(s = Cache::create(*config, batch, num_kv_heads, head_dim, &c)).ok()) return s;
    auto h = std::make_unique<kivi_oracle_cache>();
    h->c = std::move(c);
    *out = h.release();
    return Status{};
  });
}

void kivi_oracle_cache_free(kivi_oracle_cache* c) { delete c; }

kivi_config kivi_oracle_cache_config(const kivi_oracle_cache* c) { return c->c->config; }
size_t kivi_oracle_cache_batch_size(const kivi_oracle_cache* c) { return c->c->batch; }
size_t kivi_oracle_cache_num_kv_heads(const kivi_oracle_cache* c) { return c->c->heads; }
size_t kivi_oracle_cache_head_dim(const kivi_oracle_cache* c) { return c->c->head_dim; }
size_t kivi_oracle_cache_sequence_length(const kivi_oracle_cache* c) { return c->c->seq_len; }
size_t kivi_oracle_cache_key_residual_len(const kivi_oracle_cache* c) { return c->c->key_res_len; }
size_t kivi_oracle_cache_value_residual_len(const kivi_oracle_cache* c) {
  return c->c->value_res_len;
}
size_t kivi_oracle_cache_quantized_key_tokens(const kivi_oracle_cache* c) {
  return c->c->quantized_key_tokens();
}
size_t kivi_oracle_cache_quantized_value_tokens(const kivi_oracle_cache* c) {
  return c->c->quantized_value_tokens();
}
// tokens_until_key_flush / value_residual_slots_remaining (src/cache.rs:328-337).
size_t kivi_oracle_cache_tokens_until_key_flush(const kivi_oracle_cache* c) {
  const size_t r = c->c->config.residual_length;
  return r > c->c->key_res_len ? r - c->c->key_res_len : 0;
}
size_t kivi_oracle_cache_value_residual_slots_remaining(const kivi_oracle_cache* c) {
  const size_t r = c->c->config.residual_length;
  return r > c->c->value_res_len ? r - c->c->value_res_len : 0;
}

kivi_status kivi_oracle_cache_append(kivi_oracle_cache* c, const float* keys, size_t keys_len,
                                     const float* values, size_t values_len, size_t seq_len,
                                     kivi_error* err) {
  return guarded(err, [&] {
    Status s = need(c, "cache");
    if (!s.ok()) return s;
    if (!(s = need_slice(keys, keys_len, "keys")).ok()) return s;
    if (!(s = need_slice(values, values_len, "values")).ok()) return s;
    return c->c->append(keys, keys_len, values, values_len, seq_len);
  });
}

kivi_status kivi_oracle_cache_attention(const kivi_oracle_cache* c, const float* query,
                                        size_t query_len, size_t num_q_heads, float scale,
                                        float* out, size_t out_len, kivi_error* err) {
  return guarded(err, [&] {
    Status s = need(c, "cache");
    if (!s.ok()) return s;
    const Cache& cc = *c->c;
    if (num_q_heads == 0 || num_q_heads % cc.heads != 0)
      return Err(KIVI_ERR_QUERY_HEADS, num_q_heads, cc.heads);
    const size_t expected = cc.batch * num_q_heads * cc.head_dim;
    if (query_len != expected) return Err(KIVI_ERR_SHAPE, expected, query_len);
    if (out_len != expected) return Err(KIVI_ERR_SHAPE, expected, out_len);
    if (!(s = need_slice(query, query_len, "query")).ok()) return s;
    if (!(s = need_slice(out, out_len, "out")).ok()) return s;
    return cc.attention(query, query_len, num_q_heads, scale, out);
  });
}

kivi_status kivi_oracle_cache_dequantize(const kivi_oracle_cache* c, float* keys, size_t keys_len,
                                         float* values, size_t values_len, kivi_error* err) {
  return guarded(err, [&] {
    Status s = need(c, "cache");
    if (!s.ok()) return s;
    const Cache& cc = *c->c;
    const size_t n = cc.batch * cc.heads * cc.seq_len * cc.head_dim;
    if (keys_len != n) return Err(KIVI_ERR_SHAPE, n, keys_len);
    if (values_len != n) return Err(KIVI_ERR_SHAPE, n, values_len);
    if (!(s = need_slice(keys, keys_len, "keys")).ok()) return s;
    if (!(s = need_slice(values, values_len, "values")).ok()) return s;
    cc.dequantize(keys, values);
    return Status{};
  });
}

kivi_memory_report kivi_oracle_cache_memory(const kivi_oracle_cache* c) { return c->c->memory(); }

kivi_status kivi_oracle_cache_export_streams(const kivi_oracle_cache* c, uint32_t* key_codes,
                                             size_t key_codes_len, float* key_params,
                                             size_t key_params_len, uint32_t* value_codes,
                                             size_t value_codes_len, float* value_params,
                                             size_t value_params_len, kivi_error* err) {
  return guarded(err, [&] {
    Status s = need(c, "cache");
    if (!s.ok()) return s;
    const Cache& cc = *c->c;
    size_t nkc = 0, nkp = 0, nvc = 0, nvp = 0;
    for (const auto& st : cc.key_streams) {
      nkc += st.codes.size();
      nkp += st.params.size();
    }
    for (const auto& st : cc.value_streams) {
      nvc += st.codes.size();
      nvp += st.params.size();
    }
    if (key_codes && key_codes_len != nkc) return Err(KIVI_ERR_SHAPE, nkc, key_codes_len);
    if (key_params && key_params_len != nkp) return Err(KIVI_ERR_SHAPE, nkp, key_params_len);
    if (value_codes && value_codes_len != nvc) return Err(KIVI_ERR_SHAPE, nvc, value_codes_len);
    if (value_params && value_params_len != nvp)
      return Err(KIVI_ERR_SHAPE, nvp, value_params_len);
    size_t o1 = 0, o2 = 0, o3 = 0, o4 = 0;
    for (const auto& st : cc.key_streams) {
      if (key_codes) std::copy(st.codes.begin(), st.codes.end(), key_codes + o1);
      if (key_params) std::copy(st.params.begin(), st.params.end(), key_params + o2);
      o1 += st.codes.size();
      o2 += st.params.size();
    }
    for (const auto& st : cc.value_streams) {
      if (value_codes) std::copy(st.codes.begin(), st.codes.end(), value_codes + o3);
      if (value_params) std::copy(st.params.begin(), st.params.end(), value_params + o4);
      o3 += st.codes.size();
      o4 += st.params.size();
    }
    return Status{};
  });
}

kivi_status kivi_oracle_cache_reserve(kivi_oracle_cache* c, size_t tokens, kivi_error* err) {
  (void)tokens;
  return guarded(err, [&] { return need(c, "cache"); });
}

// KiviCache::share_prefix -> SharedPrefix::from_cache (src/cache.rs:178-180; src/prefix.rs:74-92).
kivi_status kivi_oracle_cache_share_prefix(const kivi_oracle_cache* c, kivi_oracle_prefix** out,
                                           kivi_error* err) {
  return guarded(err, [&] {
    Status s = need(c, "cache");
    if (!s.ok()) return s;
    if (!(s = need(out, "out")).ok()) return s;
    auto st = std::make_shared<PrefixState>();
    st->cache.config = c->c->config;
    st->cache.batch = c->c->batch;
    st->cache.heads = c->c->heads;
    st->cache.head_dim = c->c->head_dim;
    st->cache.key_streams = c->c->key_streams;
    st->cache.value_streams = c->c->value_streams;
    st->cache.key_residual = c->c->key_residual;
    st->cache.value_residual = c->c->value_residual;
    st->cache.key_res_len = c->c->key_res_len;
    st->cache.value_res_len = c->c->value_res_len;
    st->cache.seq_len = c->c->seq_len;
    st->prefix_bytes = compressed_bytes(c->c->memory());
    auto p = std::make_unique<kivi_oracle_prefix>();
    p->state = std::move(st);
    *out = p.release();
    return Status{};
  });
}

kivi_oracle_prefix* kivi_oracle_prefix_retain(kivi_oracle_prefix* p) {
  if (p == nullptr) return nullptr;
  auto q = new kivi_oracle_prefix;
  q->state = p->state;
  return q;
}
void kivi_oracle_prefix_release(kivi_oracle_prefix* p) { delete p; }

kivi_config kivi_oracle_prefix_config(const kivi_oracle_prefix* p) { return p->state->cache.config; }
size_t kivi_oracle_prefix_batch_size(const kivi_oracle_prefix* p) { return p->state->cache.batch; }
size_t kivi_oracle_prefix_num_kv_heads(const kivi_oracle_prefix* p) {
  return p->state->cache.heads;
}
size_t kivi_oracle_prefix_head_dim(const kivi_oracle_prefix* p) { return p->state->cache.head_dim; }
size_t kivi_oracle_prefix_prefix_tokens(const kivi_oracle_prefix* p) {
  return p->state->cache.seq_len;
}
size_t kivi_oracle_prefix_prefix_bytes(const kivi_oracle_prefix* p) {
  return p->state->prefix_bytes;
}
int kivi_oracle_prefix_shares_allocation_with(const kivi_oracle_prefix* a,
                                              const kivi_oracle_prefix* b) {
  return (a && b && a->state.get() == b->state.get()) ? 1 : 0;
}

// SharedPrefix::footprint (src/prefix.rs:136-152).
kivi_prefix_footprint kivi_oracle_prefix_footprint_of(const kivi_oracle_prefix* p,
                                                      size_t sessions, size_t question_tokens) {
  const Cache& st = p->state->cache;
  const size_t elements = st.batch * st.heads * st.head_dim;
  const size_t question_bytes = sessions * question_tokens * elements * 2 * 4;
  const size_t tokens = st.seq_len + question_tokens;
  const size_t fp16_per_user = 2 * tokens * elements * 2;
  kivi_prefix_footprint f{};
  f.prefix_tokens = st.seq_len;
  f.question_tokens = question_tokens;
  f.sessions = sessions;
  f.prefix_bytes = p->state->prefix_bytes;
  f.question_bytes = question_bytes;
  f.shared_total_bytes = p->state->prefix_bytes + question_bytes;
  f.fp16_per_user_bytes = fp16_per_user;
  f.fp16_all_users_bytes = sessions * fp16_per_user;
  return f;
}

// SharedPrefix::session (src/prefix.rs:124-131).
kivi_status kivi_oracle_prefix_session(kivi_oracle_prefix* p, kivi_oracle_session** out,
                                       kivi_error* err) {
  return guarded(err, [&] {
    Status s = need(p, "prefix");
    if (!s.ok()) return s;
    if (!(s = need(out, "out")).ok()) return s;
    auto ss = std::make_unique<kivi_oracle_session>();
    ss->prefix.state = p->state;
    *out = ss.release();
    return Status{};
  });
}

void kivi_oracle_session_free(kivi_oracle_session* s) { delete s; }
kivi_oracle_prefix* kivi_oracle_session_prefix(const kivi_oracle_session* s) {
  return const_cast<kivi_oracle_prefix*>(&s->prefix);
}
size_t kivi_oracle_session_prefix_tokens(const kivi_oracle_session* s) {
  return s->prefix.state->cache.seq_len;
}
size_t kivi_oracle_session_question_tokens(const kivi_oracle_session* s) { return s->local_len; }
size_t kivi_oracle_session_sequence_length(const kivi_oracle_session* s) {
  return s->prefix.state->cache.seq_len + s->local_len;
}

// RagSession::append (src/prefix.rs:173-223).
kivi_status kivi_oracle_session_append(kivi_oracle_session* s, const float* keys,
                                       size_t keys_len, const float* values, size_t values_len,
                                       size_t seq_len, kivi_error* err) {
  return guarded(err, [&] {
    Status st = need(s, "session");
    if (!st.ok()) return st;
    const Cache& c = s->prefix.state->cache;
    const size_t expected = c.batch * c.heads * seq_len * c.head_dim;
    if (keys_len != expected) return Err(KIVI_ERR_SHAPE, expected, keys_len);
    if (values_len != expected) return Err(KIVI_ERR_SHAPE, expected, values_len);
    if (seq_len == 0) return Status{};
    if (!(st = need_slice(keys, keys_len, "keys")).ok()) return st;
    if (!(st = need_slice(values, values_len, "values")).ok()) return st;
    const size_t new_len = s->local_len + seq_len;
    std::vector<float> nk(c.batch * c.heads * new_len * c.head_dim, 0.0f);
    std::vector<float> nv(c.batch * c.heads * new_len * c.head_dim, 0.0f);
    splice_tokens(nk.data(), s->local_keys.data(), keys, s->local_len, seq_len, c.batch, c.heads,
                  c.head_dim);
    splice_tokens(nv.data(), s->local_values.data(), values, s->local_len, seq_len, c.batch,
                  c.heads, c.head_dim);
    s->local_keys.swap(nk);
    s->local_values.swap(nv);
    s->local_len = new_len;
    return Status{};
  });
}

kivi_status kivi_oracle_session_attention(const kivi_oracle_session* s, const float* query,
                                          size_t query_len, size_t num_q_heads, float scale,
                                          float* out, size_t out_len, kivi_error* err) {
  return guarded(err, [&] {
    Status st = need(s, "session");
    if (!st.ok()) return st;
    const Cache& c = s->prefix.state->cache;
    if (num_q_heads == 0 || num_q_heads % c.heads != 0)
      return Err(KIVI_ERR_QUERY_HEADS, num_q_heads, c.heads);
    const size_t expected = c.batch * num_q_heads * c.head_dim;
    if (query_len != expected) return Err(KIVI_ERR_SHAPE, expected, query_len);
    if (out_len != expected) return Err(KIVI_ERR_SHAPE, expected, out_len);
    if (!(st = need_slice(query, query_len, "query")).ok()) return st;
    if (!(st = need_slice(out, out_len, "out")).ok()) return st;
    return session_attention(*s, query, query_len, num_q_heads, scale, out);
  });
}

// Batched form: by definition n independent RagSession::attention calls.
kivi_status kivi_oracle_sessions_attention(const kivi_oracle_session* const* sessions, size_t n,
                                           const float* queries, size_t queries_len,
                                           size_t num_q_heads, float scale, float* out,
                                           size_t out_len, kivi_error* err) {
  return guarded(err, [&] {
    Status st = need_slice(sessions, n, "sessions");
    if (!st.ok()) return st;
    if (n == 0) return Status{};
    const Cache& c0 = sessions[0]->prefix.state->cache;
    for (size_t i = 1; i < n; ++i)
      if (sessions[i]->prefix.state.get() != sessions[0]->prefix.state.get())
        return Err(KIVI_ERR_MISMATCHED_PREFIX, i, 0);
    if (num_q_heads == 0 || num_q_heads % c0.heads != 0)
      return Err(KIVI_ERR_QUERY_HEADS, num_q_heads, c0.heads);
    const size_t per = c0.batch * num_q_heads * c0.head_dim;
    if (queries_len != n * per) return Err(KIVI_ERR_SHAPE, n * per, queries_len);
    if (out_len != n * per) return Err(KIVI_ERR_SHAPE, n * per, out_len);
    for (size_t i = 0; i < n; ++i) {
      st = session_attention(*sessions[i], queries + i * per, per, num_q_heads, scale,
                             out + i * per);
      if (!st.ok()) return st;
    }
    return Status{};
  });
}

// RuntimeKv (src/runtime.rs:12-57).
kivi_status kivi_oracle_runtime_new(const kivi_config* config, size_t batch, size_t num_kv_heads,
                                    size_t head_dim, kivi_oracle_runtime** out, kivi_error* err) {
  if (out == nullptr) return report(Err(KIVI_ERR_NULL_ARGUMENT, 0, 0, "out"), err);
  kivi_oracle_cache* c = nullptr;
  kivi_status st = kivi_oracle_cache_new(config, batch, num_kv_heads, head_dim, &c, err);
  if (st != KIVI_OK) return st;
  auto rt = new kivi_oracle_runtime;
  rt->cache.c = std::move(c->c);
  delete c;
  *out = rt;
  return KIVI_OK;
}
void kivi_oracle_runtime_free(kivi_oracle_runtime* rt) { delete rt; }
kivi_oracle_cache* kivi_oracle_runtime_cache(kivi_oracle_runtime* rt) { return &rt->cache; }
kivi_status kivi_oracle_runtime_prefill(kivi_oracle_runtime* rt, const float* keys,
                                        size_t keys_len, const float* values, size_t values_len,
                                        size_t seq_len, kivi_error* err) {
  return kivi_oracle_cache_append(&rt->cache, keys, keys_len, values, values_len, seq_len, err);
}
kivi_status kivi_oracle_runtime_decode(kivi_oracle_runtime* rt, const float* key, size_t key_len,
                                       const float* value, size_t value_len, const float* query,
                                       size_t query_len, size_t num_q_heads, float scale,
                                       float* out, size_t out_len, kivi_error* err) {
  kivi_status st = kivi_oracle_cache_append(&rt->cache, key, key_len, value, value_len, 1, err);
  if (st != KIVI_OK) return st;
  return kivi_oracle_cache_attention(&rt->cache, query, query_len, num_q_heads, scale, out,
                                     out_len, err);
}

// QualityGuard::try_new and accessors (src/guard.rs:50-88).
kivi_status kivi_oracle_guard_new(const kivi_config* config, size_t batch, size_t num_kv_heads,
                                  size_t head_dim, float threshold, uint32_t policy,
                                  uint8_t max_bits, size_t max_residual, kivi_oracle_guard** out,
                                  kivi_error* err) {
  return guarded(err, [&] {
    Status s = need(config, "config");
    if (!s.ok()) return s;
    if (!(s = need(out, "out")).ok()) return s;
    if (policy != KIVI_POLICY_RAISE_BITS && policy != KIVI_POLICY_LENGTHEN_RESIDUAL)
      return Err(KIVI_ERR_UNSUPPORTED, policy, 1, "policy");
    if (!(s = config_try_new(config->bits, config->group_size, config->residual_length)).ok())
      return s;
    auto g = std::make_unique<kivi_oracle_guard>();
    if (!(s = Cache::create(*config, batch, num_kv_heads, head_dim, &g->cache.c)).ok()) return s;
    g->threshold = threshold;
    g->policy = policy;
    g->max_bits = max_bits;
    g->max_residual = max_residual;
    *out = g.release();
    return Status{};
  });
}
void kivi_oracle_guard_free(kivi_oracle_guard* g) { delete g; }
kivi_config kivi_oracle_guard_config(const kivi_oracle_guard* g) { return g->cache.c->config; }
uint32_t kivi_oracle_guard_policy(const kivi_oracle_guard* g) { return g->policy; }
size_t kivi_oracle_guard_sequence_length(const kivi_oracle_guard* g) { return g->seq; }
kivi_oracle_cache* kivi_oracle_guard_cache(kivi_oracle_guard* g) { return g ? &g->cache : nullptr; }

// QualityGuard::append / check / propose (src/guard.rs:90-193).
kivi_status kivi_oracle_guard_append(kivi_oracle_guard* g, const float* keys, size_t keys_len,
                                     const float* values, size_t values_len, size_t seq_len,
                                     const float* query, size_t query_len, size_t num_q_heads,
                                     float scale, kivi_flush_check* checks, size_t checks_cap,
                                     size_t* num_checks, kivi_error* err) {
  return guarded(err, [&]() -> Status {
    Status s = need(g, "guard");
    if (!s.ok()) return s;
    const size_t batch = g->cache.c->batch, heads = g->cache.c->heads, dim = g->cache.c->head_dim;
    const size_t expected = batch * heads * seq_len * dim;
    if (keys_len != expected) return Err(KIVI_ERR_SHAPE, expected, keys_len);
    if (values_len != expected) return Err(KIVI_ERR_SHAPE, expected, values_len);
    const size_t query_elems = batch * num_q_heads * dim;
    if (num_q_heads == 0 || num_q_heads % heads != 0)
      return Err(KIVI_ERR_QUERY_HEADS, num_q_heads, heads);
    if (query_len != query_elems) return Err(KIVI_ERR_SHAPE, query_elems, query_len);
    if (!(s = need_slice(query, query_len, "query")).ok()) return s;
    if (!(s = need_slice(keys, keys_len, "keys")).ok()) return s;
    if (!(s = need_slice(values, values_len, "values")).ok()) return s;
    if (checks_cap > 0 && !(s = need(checks, "checks")).ok()) return s;
    if (!(s = need(num_checks, "num_checks")).ok()) return s;
    g->last.clear();
    size_t offset = 0;
    while (offset < seq_len) {
      const size_t r = g->cache.c->config.residual_length;
      const size_t room = r > g->cache.c->key_res_len ? r - g->cache.c->key_res_len : 0;
      const size_t take = room < seq_len - offset ? room : seq_len - offset;
      const std::vector<float> ks = guard_slice(keys, batch, heads, seq_len, offset, take, dim);
      const std::vector<float> vs = guard_slice(values, batch, heads, seq_len, offset, take, dim);
      if (!(s = g->cache.c->append(ks.data(), ks.size(), vs.data(), vs.size(), take)).ok()) return s;
      // push_history (src/guard.rs:237-245)
      g->keys = guard_concat(g->keys, ks, g->seq, take, batch, heads, dim);
      g->values = guard_concat(g->values, vs, g->seq, take, batch, heads, dim);
      g->seq += take;
      if (g->cache.c->key_res_len == 0) {
        kivi_flush_check fc{};
        if (!(s = guard_cosine(*g, query, query_len, num_q_heads, scale, &fc.cosine_before)).ok())
          return s;
        fc.cosine = fc.cosine_before;
        while (fc.cosine < g->threshold) {
          const kivi_config cfg = g->cache.c->config;
          kivi_quality_upgrade up{};
          if (g->policy == KIVI_POLICY_RAISE_BITS) {
            uint8_t to;
            if (!guard_next_bits(cfg.bits, g->max_bits, &to)) break;
            up = kivi_quality_upgrade{0, cfg.bits, to};
          } else {
            size_t to;
            if (!guard_next_residual(cfg.residual_length, cfg.group_size, g->max_residual, &to)) break;
            up = kivi_quality_upgrade{1, cfg.residual_length, to};
          }
          if (fc.num_upgrades == KIVI_MAX_UPGRADES)
            return Err(KIVI_ERR_CAPACITY, fc.num_upgrades + 1, KIVI_MAX_UPGRADES, "upgrades");
          if (!(s = guard_apply(*g, up)).ok()) return s;
          fc.upgrades[fc.num_upgrades++] = up;
          if (!(s = guard_cosine(*g, query, query_len, num_q_heads, scale, &fc.cosine)).ok()) return s;
        }
        fc.sequence_tokens = g->seq;
        g->last.push_back(fc);
      }
      offset += take;
    }
    *num_checks = g->last.size();
    for (size_t i = 0; i < g->last.size() && i < checks_cap; ++i) checks[i] = g->last[i];
    return Status{};
  });
}

size_t kivi_oracle_guard_last_checks(const kivi_oracle_guard* g, size_t first,
                                     kivi_flush_check* checks, size_t cap) {
  if (g == nullptr || checks == nullptr) return 0;
  size_t n = 0;
  for (size_t i = first; i < g->last.size() && n < cap; ++i) checks[n++] = g->last[i];
  return n;
}

// fp32_attention (src/guard.rs:344-385) over [batch*kv_heads][seq][dim] rows, for the tests.
void kivi_oracle_fp32_attention(const float* query, const float* keys, const float* values,
                                size_t batch, size_t kv_heads, size_t q_heads, size_t seq,
                                size_t dim, float scale, float* out) {
  const size_t n = batch * kv_heads * seq * dim;
  const std::vector<float> k(keys, keys + n), v(values, values + n);
  const std::vector<float> o =
      guard_fp32_attention(query, k, v, batch, kv_heads, q_heads, seq, dim, scale);
  std::memcpy(out, o.data(), o.size() * 4);
}

// quantize_per_channel / quantize_per_token (src/quant.rs:153-233).
kivi_status kivi_oracle_quantize_per_channel(const float* data, size_t data_len, size_t batch,
                                             size_t heads, size_t tokens, size_t head_dim,
                                             uint8_t bits, size_t group_size,
                                             kivi_oracle_quantized** out, kivi_error* err) {
  return guarded(err, [&] {
    return quantize_impl(data, data_len, batch, heads, tokens, head_dim, bits, group_size, true,
                         out);
  });
}
kivi_status kivi_oracle_quantize_per_token(const float* data, size_t data_len, size_t batch,
                                           size_t heads, size_t tokens, size_t head_dim,
                                           uint8_t bits, size_t group_size,
                                           kivi_oracle_quantized** out, kivi_error* err) {
  return guarded(err, [&] {
    return quantize_impl(data, data_len, batch, heads, tokens, head_dim, bits, group_size, false,
                         out);
  });
}
void kivi_oracle_quantized_free(kivi_oracle_quantized* q) { delete q; }
int kivi_oracle_quantized_axis(const kivi_oracle_quantized* q) { return q->axis; }
uint8_t kivi_oracle_quantized_bits(const kivi_oracle_quantized* q) { return q->bits; }
size_t kivi_oracle_quantized_group_size(const kivi_oracle_quantized* q) { return q->group_size; }
size_t kivi_oracle_quantized_num_tokens(const kivi_oracle_quantized* q) { return q->tokens; }
// code_bytes / metadata_bytes (src/quant.rs:63-69).
size_t kivi_oracle_quantized_code_bytes(const kivi_oracle_quantized* q) {
  size_t n = 0;
  for (const auto& s : q->streams) n += s.codes.size() * 4;
  return n;
}
size_t kivi_oracle_quantized_metadata_bytes(const kivi_oracle_quantized* q) {
  size_t n = 0;
  for (const auto& s : q->streams) n += s.params.size() * 4;
  return n;
}

kivi_status kivi_oracle_quantized_codes(const kivi_oracle_quantized* q, uint32_t* out,
                                        size_t out_len, kivi_error* err) {
  return guarded(err, [&] {
    const size_t n = kivi_oracle_quantized_code_bytes(q) / 4;
    if (out_len != n) return Err(KIVI_ERR_SHAPE, n, out_len);
    size_t o = 0;
    for (const auto& s : q->streams) {
      std::copy(s.codes.begin(), s.codes.end(), out + o);
      o += s.codes.size();
    }
    return Status{};
  });
}

// QuantizedTensor::pytorch_codes (src/quant.rs:77-112).
kivi_status kivi_oracle_quantized_pytorch_codes(const kivi_oracle_quantized* q, uint32_t* out,
                                                size_t out_len, kivi_error* err) {
  return guarded(err, [&] {
    const size_t n = kivi_oracle_quantized_code_bytes(q) / 4;
    if (out_len != n) return Err(KIVI_ERR_SHAPE, n, out_len);
    const size_t feat = 32 / q->bits;
    size_t o = 0;
    if (q->axis == KIVI_AXIS_PER_CHANNEL) {
      const size_t t_pack = q->tokens / feat;
      const size_t ipc = q->group_size * q->bits / 32;
      for (const auto& s : q->streams)
        for (size_t tp = 0; tp < t_pack; ++tp) {
          const size_t g = tp / ipc, w = tp % ipc;
          for (size_t d = 0; d < q->head_dim; ++d) out[o++] = s.codes[(g * q->head_dim + d) * ipc + w];
        }
    } else {
      const size_t n_ch = q->head_dim / q->group_size;
      const size_t ipg = q->group_size * q->bits / 32;
      const size_t d_pack = q->head_dim / feat;
      for (const auto& s : q->streams)
        for (size_t t = 0; t < q->tokens; ++t)
          for (size_t dp = 0; dp < d_pack; ++dp) {
            const size_t cg = dp / ipg, w = dp % ipg;
            out[o++] = s.codes[(t * n_ch + cg) * ipg + w];
          }
    }
    return Status{};
  });
}

// QuantizedTensor::scale_zero (src/quant.rs:116-121).
kivi_status kivi_oracle_quantized_scale_zero(const kivi_oracle_quantized* q, float* out,
                                             size_t out_len, kivi_error* err) {
  return guarded(err, [&] {
    const size_t n = kivi_oracle_quantized_metadata_bytes(q) / 4;
    if (out_len != n) return Err(KIVI_ERR_SHAPE, n, out_len);
    size_t o = 0;
    for (const auto& s : q->streams) {
      std::copy(s.params.begin(), s.params.end(), out + o);
      o += s.params.size();
    }
    return Status{};
  });
}

// QuantizedTensor::dequantize (src/quant.rs:124-150).
kivi_status kivi_oracle_quantized_dequantize(const kivi_oracle_quantized* q, float* out,
                                             size_t out_len, kivi_error* err) {
  return guarded(err, [&] {
    const size_t n = q->batch * q->heads * q->tokens * q->head_dim;
    if (out_len != n) return Err(KIVI_ERR_SHAPE, n, out_len);
    std::fill(out, out + n, 0.0f);
    for (size_t b = 0; b < q->batch; ++b)
      for (size_t h = 0; h < q->heads; ++h) {
        const size_t hi = b * q->heads + h;
        float* dst = out + hi * q->tokens * q->head_dim;
        if (q->axis == KIVI_AXIS_PER_CHANNEL)
          dequant_keys(q->streams[hi], q->bits, q->group_size, q->head_dim, dst);
        else
          dequant_values(q->streams[hi], q->bits, q->group_size, q->head_dim, dst);
      }
    return Status{};
  });
}

// round_half_even exposed for the rounding tests (src/quant.rs:475-485).
float kivi_oracle_round_half_even(float x) { return round_half_even(x); }

int32_t kivi_oracle_abi_version(void) { return KIVI_ABI_VERSION; }

}  // extern "C"
