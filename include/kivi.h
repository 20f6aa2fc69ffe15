/*
 * kivi.h — C ABI of the MI355X-native KIVI KV cache (libkivi_amd.so).
 *
 * This is the drop-in boundary for the hot path of bieli/kivi-cache-rs v0.6.0:
 * KIVI 2/4/8-bit KV-cache quantization plus fused decode attention, behind the
 * reference's KiviCache / SharedPrefix / RagSession / RuntimeKv / quantize_* API.
 * Every entry point below names the reference item it replaces (file:line in the
 * reference crate). A Rust, C or Python host binds these symbols directly; no
 * framework type crosses the boundary (plain pointers, sizes and POD structs).
 *
 * Conventions
 *  - Dense tensors are row-major f32: keys/values [batch, num_kv_heads, seq, head_dim],
 *    queries/outputs [batch, num_q_heads, head_dim]  (reference src/cache.rs:60-63, 216-223).
 *  - Every fallible call returns a kivi_status and, when `err` is non-NULL, fills it
 *    with the variant payload and the reference's Display text (src/error.rs:47-95).
 *    Checks run in the reference's order, so the first error reported is the one the
 *    reference would report.
 *  - Lengths are passed explicitly so Shape{expected, actual} is reproducible: the
 *    reference's `&[f32]` becomes (pointer, element count).
 *  - Results the reference returns as a fresh Vec are written to a caller buffer
 *    whose element count is passed too (a wrong count is a Shape error).
 *  - Host-pointer entry points are synchronous: on return the caller's buffers may be
 *    reused and outputs are complete. `*_device` entry points take device pointers and
 *    a hipStream_t (as void*), enqueue work on that stream and return without waiting.
 *    Attention calls on one cache (or one session) reuse its device workspace: a call on
 *    a different stream than the previous one first waits for the previous stream's work,
 *    so that stream must still exist then (or the cache / session must be freed first).
 *    A host-pointer call on a cache (and kivi_cache_reserve, kivi_cache_share_prefix and
 *    freeing the cache) first waits for the stream of the latest `*_device` call on it when
 *    that is not the cache's own stream (kivi_cache_set_stream), and a host-pointer call on
 *    a session for that of the latest `*_device` call on the session when it is not the
 *    default stream, so it never overlaps that work; that stream must still exist then too.
 *    Likewise the host reads of a QuantizedTensor made by kivi_quantize_*_device wait for
 *    the stream of that call first.
 *    Calls enqueued under stream capture are not counted. Between `*_device` calls on
 *    different streams the caller orders the work.
 *  - Threading follows the reference's borrow rules: at most one mutating call
 *    (append, reserve, prefill, decode) in flight per cache; read-only calls
 *    (attention, dequantize, export, getters) may share a cache but must not overlap
 *    a mutating call. Prefix handles are reference counted and may be shared by
 *    sessions on any thread.
 *  - There is no CPU fallback: without a usable HIP device the compute entry points
 *    return KIVI_ERR_DEVICE.
 */
#ifndef KIVI_AMD_H
#define KIVI_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KIVI_ABI_VERSION 1

/* ---------------------------------------------------------------- status */

/* Mirrors enum KiviError (reference src/error.rs:5-45), variant order preserved. */
typedef enum kivi_status {
  KIVI_OK = 0,
  KIVI_ERR_INVALID_BITS = 1,      /* InvalidBits(bits):                      a = bits */
  KIVI_ERR_MISALIGNED_GROUP = 2,  /* MisalignedGroup{group_size, bits}:      a, b */
  KIVI_ERR_RESIDUAL_LENGTH = 3,   /* ResidualLength{residual_length, group_size}: a, b */
  KIVI_ERR_HEAD_DIM = 4,          /* HeadDim{head_dim, group_size}:          a, b */
  KIVI_ERR_TOKEN_GROUP = 5,       /* TokenGroup{tokens, group_size}:         a, b */
  KIVI_ERR_ZERO_DIMENSION = 6,    /* ZeroDimension(name):                    name */
  KIVI_ERR_SHAPE = 7,             /* Shape{expected, actual}:                a, b */
  KIVI_ERR_QUERY_HEADS = 8,       /* QueryHeads{num_q_heads, num_kv_heads}:  a, b */
  KIVI_ERR_EARLY_LAYERS = 9,      /* EarlyLayers{early_layers, num_layers}: planner only, never returned here */
  /* Extensions with no reference counterpart. */
  KIVI_ERR_NULL_ARGUMENT = 100,   /* a required pointer was NULL (name) */
  KIVI_ERR_DEVICE = 101,          /* HIP runtime failure or no device (message) */
  KIVI_ERR_CAPACITY = 102,        /* size overflow or a size beyond a documented limit */
  KIVI_ERR_UNSUPPORTED = 103,     /* valid for the reference, outside this build's limits */
  KIVI_ERR_MISMATCHED_PREFIX = 104 /* batched sessions do not share one prefix */
} kivi_status;

typedef struct kivi_error {
  int32_t code;          /* kivi_status */
  uint64_t a;            /* first payload field (see kivi_status) */
  uint64_t b;            /* second payload field */
  char name[32];         /* ZeroDimension / NullArgument field name */
  char message[192];     /* Display text, NUL terminated */
} kivi_error;

/* ---------------------------------------------------------------- config */

/* KiviConfig (reference src/config.rs:9-18). */
typedef struct kivi_config {
  uint8_t bits;             /* 2, 4 or 8 */
  size_t group_size;        /* tokens per key group, channels per value group */
  size_t residual_length;   /* fp32 window R (keys flush every R tokens) */
} kivi_config;

/* KiviConfig::default() = {2, 32, 128} (src/config.rs:20-28). */
void kivi_config_default(kivi_config* out);

/* KiviConfig::try_new (src/config.rs:31-45; check order src/config.rs:47-54). */
kivi_status kivi_config_try_new(uint8_t bits, size_t group_size, size_t residual_length,
                                kivi_config* out, kivi_error* err);

/* ---------------------------------------------------------------- reports */

/* MemoryReport (src/cache.rs:25-36). */
typedef struct kivi_memory_report {
  size_t tokens;
  size_t key_code_bytes;
  size_t key_metadata_bytes;
  size_t value_code_bytes;
  size_t value_metadata_bytes;
  size_t key_residual_bytes;
  size_t value_residual_bytes;
  size_t residual_capacity_bytes;
  size_t fp16_baseline_bytes;
  size_t fp32_baseline_bytes;
} kivi_memory_report;

/* MemoryReport::compressed_bytes / compression_ratio_vs_fp16 (src/cache.rs:40-57). */
size_t kivi_memory_compressed_bytes(const kivi_memory_report* r);
double kivi_memory_compression_ratio_vs_fp16(const kivi_memory_report* r);

/* SharedPrefixFootprint (src/prefix.rs:51-60). */
typedef struct kivi_prefix_footprint {
  size_t prefix_tokens;
  size_t question_tokens;
  size_t sessions;
  size_t prefix_bytes;
  size_t question_bytes;
  size_t shared_total_bytes;
  size_t fp16_per_user_bytes;
  size_t fp16_all_users_bytes;
} kivi_prefix_footprint;

/* SharedPrefixFootprint::savings_vs_fp16 (src/prefix.rs:62-71). */
double kivi_footprint_savings_vs_fp16(const kivi_prefix_footprint* f);

/* ---------------------------------------------------------------- cache */

typedef struct kivi_cache kivi_cache;

/* KiviCache::new (src/cache.rs:87-120): checks batch, num_kv_heads, then head_dim.
 * The config is validated first as KiviConfig::try_new would (the reference trusts
 * its pub fields; an unvalidated residual_length of 0 loops forever there). */
kivi_status kivi_cache_new(const kivi_config* config, size_t batch, size_t num_kv_heads,
                           size_t head_dim, kivi_cache** out, kivi_error* err);
void kivi_cache_free(kivi_cache* cache);

/* Stream used by the host-pointer entry points and by internal copies
 * (hipStream_t as void*; NULL = the default stream). Switching waits for the work enqueued
 * on the previous stream (and for the latest `*_device` call's stream) first, so the
 * previous stream must still exist then. */
kivi_status kivi_cache_set_stream(kivi_cache* cache, void* stream, kivi_error* err);

/* Getters (src/cache.rs:122-156, 328-337). */
kivi_config kivi_cache_config(const kivi_cache* cache);
size_t kivi_cache_batch_size(const kivi_cache* cache);
size_t kivi_cache_num_kv_heads(const kivi_cache* cache);
size_t kivi_cache_head_dim(const kivi_cache* cache);
size_t kivi_cache_sequence_length(const kivi_cache* cache);
size_t kivi_cache_key_residual_len(const kivi_cache* cache);
size_t kivi_cache_value_residual_len(const kivi_cache* cache);
size_t kivi_cache_quantized_key_tokens(const kivi_cache* cache);
size_t kivi_cache_quantized_value_tokens(const kivi_cache* cache);
size_t kivi_cache_tokens_until_key_flush(const kivi_cache* cache);
size_t kivi_cache_value_residual_slots_remaining(const kivi_cache* cache);

/* KiviCache::append (src/cache.rs:186-214): keys length then values length are
 * checked (Shape), seq_len == 0 is a no-op. Host pointers, synchronous. */
kivi_status kivi_cache_append(kivi_cache* cache, const float* keys, size_t keys_len,
                              const float* values, size_t values_len, size_t seq_len,
                              kivi_error* err);
/* Same, device pointers, enqueued on `stream`. */
kivi_status kivi_cache_append_device(kivi_cache* cache, const float* keys, size_t keys_len,
                                     const float* values, size_t values_len, size_t seq_len,
                                     void* stream, kivi_error* err);

/* KiviCache::attention (src/cache.rs:224-279): QueryHeads is checked before the
 * query Shape; an empty cache yields zeros. `out` holds batch*num_q_heads*head_dim
 * floats (a different out_len is a Shape error reported after the query checks). */
kivi_status kivi_cache_attention(const kivi_cache* cache, const float* query, size_t query_len,
                                 size_t num_q_heads, float scale, float* out, size_t out_len,
                                 kivi_error* err);
kivi_status kivi_cache_attention_device(const kivi_cache* cache, const float* query,
                                        size_t query_len, size_t num_q_heads, float scale,
                                        float* out, size_t out_len, void* stream,
                                        kivi_error* err);
/* No counterpart in the reference. For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): the same attention
 * as kivi_cache_attention_device, bit for bit, with its split partials in a static workspace
 * the library holds on each device until the process ends (2,097,152 floats = 8 MiB; the
 * partials of one call are units * splits * (num_q_heads/num_kv_heads) * (head_dim + 2)
 * floats, about 1.26 M for batch 16 x 8 KV heads x 32768 tokens with 32 query heads). It calls
 * no hipMalloc, hipFree or memset (an empty cache's zeros come from a fill kernel) and does not
 * wait for the device. Larger calls return KIVI_ERR_CAPACITY (a = floats needed, b = the
 * limit). Every call on one device shares that device's workspace. Calls on one stream are
 * ordered by the stream; a call on another stream than the previous call waits (on the device,
 * through an event the library creates once per device at its first call there) for the work
 * enqueued on that stream so far. A call made under stream capture is ordered only by the
 * stream its graph is launched on: graph launches that overlap other calls on the device
 * race, and ordering them is the caller's part. */
kivi_status kivi_cache_attention_device_noalloc(const kivi_cache* cache, const float* query,
                                                size_t query_len, size_t num_q_heads, float scale,
                                                float* out, size_t out_len, void* stream,
                                                kivi_error* err);

/* KiviCache::dequantize (src/cache.rs:282-325): both outputs hold
 * batch*num_kv_heads*seq*head_dim floats. */
kivi_status kivi_cache_dequantize(const kivi_cache* cache, float* keys, size_t keys_len,
                                  float* values, size_t values_len, kivi_error* err);
/* Same, into device buffers, enqueued on `stream` (hipStream_t as void*). */
kivi_status kivi_cache_dequantize_device(const kivi_cache* cache, float* keys, size_t keys_len,
                                         float* values, size_t values_len, void* stream,
                                         kivi_error* err);

/* KiviCache::memory (src/cache.rs:362-380). */
kivi_memory_report kivi_cache_memory(const kivi_cache* cache);

/* Packed streams in the reference's PackedStream order (src/quant.rs:37-44,
 * 307-323, 349-375), concatenated over (batch, kv_head) — the parity read-out.
 * Lengths per stream: key codes kq*D*bits/32, key params 2*(kq/G)*D,
 * value codes vq*D*bits/32, value params 2*vq*(D/G). Any pointer may be NULL
 * to skip that array; a non-NULL array with the wrong length is a Shape error. */
kivi_status kivi_cache_export_streams(const kivi_cache* cache, uint32_t* key_codes,
                                      size_t key_codes_len, float* key_params,
                                      size_t key_params_len, uint32_t* value_codes,
                                      size_t value_codes_len, float* value_params,
                                      size_t value_params_len, kivi_error* err);
/* Same, into device buffers, enqueued on `stream`. */
kivi_status kivi_cache_export_streams_device(const kivi_cache* cache, uint32_t* key_codes,
                                             size_t key_codes_len, float* key_params,
                                             size_t key_params_len, uint32_t* value_codes,
                                             size_t value_codes_len, float* value_params,
                                             size_t value_params_len, void* stream,
                                             kivi_error* err);

/* Extension: pre-size the device arenas for `tokens` total tokens per sequence so
 * later appends never reallocate (the reference's Vec::reserve, src/quant.rs:291-292). */
kivi_status kivi_cache_reserve(kivi_cache* cache, size_t tokens, kivi_error* err);

/* Extension, arena sizing (the device counterpart of the byte model of src/budget.rs:317-347,
   which counts occupied bytes): HBM a cache holds, packed arenas at their capacity plus the
   fp32 key residual and value window and the per-unit scale maxima (attention scratch, sized
   per call, is not counted). kivi_cache_device_bytes reads a live cache; kivi_plan_device_bytes
   gives what a cache of that shape holds after kivi_cache_reserve(tokens) (config checked as
   kivi_cache_new checks it). */
size_t kivi_cache_device_bytes(const kivi_cache* cache);
kivi_status kivi_plan_device_bytes(const kivi_config* config, size_t batch, size_t num_kv_heads,
                                   size_t head_dim, size_t tokens, size_t* out, kivi_error* err);

/* ---------------------------------------------------------------- prefix / sessions */

typedef struct kivi_prefix kivi_prefix;
typedef struct kivi_session kivi_session;

/* KiviCache::share_prefix -> SharedPrefix::from_cache (src/cache.rs:178-180,
 * src/prefix.rs:74-92): a frozen device copy; the returned handle holds one reference. */
kivi_status kivi_cache_share_prefix(const kivi_cache* cache, kivi_prefix** out, kivi_error* err);
/* SharedPrefix::clone (Arc clone) and drop. */
kivi_prefix* kivi_prefix_retain(kivi_prefix* prefix);
void kivi_prefix_release(kivi_prefix* prefix);

/* SharedPrefix accessors (src/prefix.rs:94-122). */
kivi_config kivi_prefix_config(const kivi_prefix* prefix);
size_t kivi_prefix_batch_size(const kivi_prefix* prefix);
size_t kivi_prefix_num_kv_heads(const kivi_prefix* prefix);
size_t kivi_prefix_head_dim(const kivi_prefix* prefix);
size_t kivi_prefix_prefix_tokens(const kivi_prefix* prefix);
size_t kivi_prefix_prefix_bytes(const kivi_prefix* prefix);
int kivi_prefix_shares_allocation_with(const kivi_prefix* a, const kivi_prefix* b);
/* SharedPrefix::footprint (src/prefix.rs:136-152). */
kivi_prefix_footprint kivi_prefix_footprint_of(const kivi_prefix* prefix, size_t sessions,
                                               size_t question_tokens);

/* SharedPrefix::session (src/prefix.rs:124-131). */
kivi_status kivi_prefix_session(kivi_prefix* prefix, kivi_session** out, kivi_error* err);
void kivi_session_free(kivi_session* session);
/* RagSession::prefix (borrowed, valid while the session lives) and getters (src/prefix.rs:155-170). */
kivi_prefix* kivi_session_prefix(const kivi_session* session);
size_t kivi_session_prefix_tokens(const kivi_session* session);
size_t kivi_session_question_tokens(const kivi_session* session);
size_t kivi_session_sequence_length(const kivi_session* session);

/* RagSession::append (src/prefix.rs:173-223): shapes first, then seq_len == 0 is a no-op. */
kivi_status kivi_session_append(kivi_session* session, const float* keys, size_t keys_len,
                                const float* values, size_t values_len, size_t seq_len,
                                kivi_error* err);
kivi_status kivi_session_append_device(kivi_session* session, const float* keys,
                                       size_t keys_len, const float* values, size_t values_len,
                                       size_t seq_len, void* stream, kivi_error* err);

/* RagSession::attention (src/prefix.rs:228-289). */
kivi_status kivi_session_attention(const kivi_session* session, const float* query,
                                   size_t query_len, size_t num_q_heads, float scale, float* out,
                                   size_t out_len, kivi_error* err);

/* Extension, no reference counterpart: n sessions of ONE prefix scored in one pass
 * that streams each prefix tile from HBM once for all of them (one launch per 64
 * sessions). Semantically sessions[i].attention(queries[i]) for every i
 * (src/prefix.rs:228-289). queries/out are [n][batch][num_q_heads][head_dim]. Device
 * pointers for queries/out, enqueued on `stream`. The split workspace belongs to the
 * prefix: batched calls on one prefix are ordered after each other (a call on another
 * stream waits for the previous call's stream, which must still exist). The sessions'
 * suffixes must not be appended to while a call that reads them is in flight. */
kivi_status kivi_sessions_attention_device(const kivi_session* const* sessions, size_t n,
                                           const float* queries, size_t queries_len,
                                           size_t num_q_heads, float scale, float* out,
                                           size_t out_len, void* stream, kivi_error* err);
/* Same with host pointers, synchronous. */
kivi_status kivi_sessions_attention(const kivi_session* const* sessions, size_t n,
                                    const float* queries, size_t queries_len,
                                    size_t num_q_heads, float scale, float* out, size_t out_len,
                                    kivi_error* err);

/* ---------------------------------------------------------------- runtime adapter */

typedef struct kivi_runtime kivi_runtime;

/* RuntimeKv::try_new / cache / prefill / decode (src/runtime.rs:16-56). */
kivi_status kivi_runtime_new(const kivi_config* config, size_t batch, size_t num_kv_heads,
                             size_t head_dim, kivi_runtime** out, kivi_error* err);
void kivi_runtime_free(kivi_runtime* rt);
kivi_cache* kivi_runtime_cache(kivi_runtime* rt);
kivi_status kivi_runtime_prefill(kivi_runtime* rt, const float* keys, size_t keys_len,
                                 const float* values, size_t values_len, size_t seq_len,
                                 kivi_error* err);
/* append(key, value, 1) then attention(query) (src/runtime.rs:46-56). */
kivi_status kivi_runtime_decode(kivi_runtime* rt, const float* key, size_t key_len,
                                const float* value, size_t value_len, const float* query,
                                size_t query_len, size_t num_q_heads, float scale, float* out,
                                size_t out_len, kivi_error* err);
/* The same on device pointers, enqueued on `stream` (inputs read by the enqueued work). A step
   without a key flush due runs, at head_dim 128, G = 32 and up to eight query heads per KV head,
   as one attention launch that carries the append, plus the merge launch; other steps run as
   the append and then the attention. Either way the result is bit for bit that of append then
   attention. */
kivi_status kivi_runtime_decode_device(kivi_runtime* rt, const float* key, size_t key_len,
                                       const float* value, size_t value_len, const float* query,
                                       size_t query_len, size_t num_q_heads, float scale,
                                       float* out, size_t out_len, void* stream,
                                       kivi_error* err);

/* ---------------------------------------------------------------- QualityGuard */
/* QualityGuard (src/guard.rs:37-258): a cache plus the fp32 tape of every appended token;
   after each key flush the guard scores cache attention against fp32 attention over the tape
   (cosine) and, below the threshold, rebuilds the cache from the tape with wider codes or a
   longer residual window. */
typedef struct kivi_guard kivi_guard;

/* QualityPolicy (src/guard.rs:13-19). */
enum { KIVI_POLICY_RAISE_BITS = 0, KIVI_POLICY_LENGTHEN_RESIDUAL = 1 };

/* QualityUpgrade (src/guard.rs:22-26): kind 0 = Bits{from, to}, 1 = Residual{from, to}. */
typedef struct kivi_quality_upgrade {
  uint32_t kind;
  size_t from;
  size_t to;
} kivi_quality_upgrade;

#define KIVI_MAX_UPGRADES 64
/* FlushCheck (src/guard.rs:29-35); upgrades[0 .. num_upgrades). */
typedef struct kivi_flush_check {
  size_t sequence_tokens;
  float cosine_before;
  float cosine;
  size_t num_upgrades;
  kivi_quality_upgrade upgrades[KIVI_MAX_UPGRADES];
} kivi_flush_check;

/* QualityGuard::try_new (src/guard.rs:51-73). */
kivi_status kivi_guard_new(const kivi_config* config, size_t batch, size_t num_kv_heads,
                           size_t head_dim, float threshold, uint32_t policy, uint8_t max_bits,
                           size_t max_residual, kivi_guard** out, kivi_error* err);
void kivi_guard_free(kivi_guard* guard);
/* config / cache / policy / sequence_length (src/guard.rs:75-88); the cache is borrowed and
   replaced by a rebuild. */
kivi_config kivi_guard_config(const kivi_guard* guard);
kivi_cache* kivi_guard_cache(kivi_guard* guard);
uint32_t kivi_guard_policy(const kivi_guard* guard);
size_t kivi_guard_sequence_length(const kivi_guard* guard);
/* QualityGuard::append (src/guard.rs:90-146), checked in the reference order (keys, values,
   query heads, query). One check per key flush inside the append: *num_checks gets their
   count and checks[0 .. min(count, checks_cap)) the first of them (checks may be NULL when
   checks_cap is 0). The guard keeps every check of its last append until the next one. */
kivi_status kivi_guard_append(kivi_guard* guard, const float* keys, size_t keys_len,
                              const float* values, size_t values_len, size_t seq_len,
                              const float* query, size_t query_len, size_t num_q_heads,
                              float scale, kivi_flush_check* checks, size_t checks_cap,
                              size_t* num_checks, kivi_error* err);
/* Checks [first, first + cap) of the last append (fewer at its end) into `checks`; returns
   how many were written. No counterpart in the reference, whose append returns a Vec. */
size_t kivi_guard_last_checks(const kivi_guard* guard, size_t first, kivi_flush_check* checks,
                              size_t cap);

/* ---------------------------------------------------------------- standalone codec */

typedef struct kivi_quantized kivi_quantized;

typedef enum kivi_quant_axis {
  KIVI_AXIS_PER_CHANNEL = 0,  /* QuantAxis::PerChannel (keys) */
  KIVI_AXIS_PER_TOKEN = 1     /* QuantAxis::PerToken (values) */
} kivi_quant_axis;

/* quantize_per_channel / quantize_per_token (src/quant.rs:153-233; argument checks
 * in the order of check_quant_args, src/quant.rs:235-273). Host data, synchronous. */
kivi_status kivi_quantize_per_channel(const float* data, size_t data_len, size_t batch,
                                      size_t heads, size_t tokens, size_t head_dim, uint8_t bits,
                                      size_t group_size, kivi_quantized** out, kivi_error* err);
kivi_status kivi_quantize_per_token(const float* data, size_t data_len, size_t batch,
                                    size_t heads, size_t tokens, size_t head_dim, uint8_t bits,
                                    size_t group_size, kivi_quantized** out, kivi_error* err);
/* Device-data variants (data stays on the device), enqueued on `stream`. */
kivi_status kivi_quantize_per_channel_device(const float* data, size_t data_len, size_t batch,
                                             size_t heads, size_t tokens, size_t head_dim,
                                             uint8_t bits, size_t group_size, void* stream,
                                             kivi_quantized** out, kivi_error* err);
kivi_status kivi_quantize_per_token_device(const float* data, size_t data_len, size_t batch,
                                           size_t heads, size_t tokens, size_t head_dim,
                                           uint8_t bits, size_t group_size, void* stream,
                                           kivi_quantized** out, kivi_error* err);
void kivi_quantized_free(kivi_quantized* q);

/* QuantizedTensor accessors (src/quant.rs:46-69). */
int kivi_quantized_axis(const kivi_quantized* q);
uint8_t kivi_quantized_bits(const kivi_quantized* q);
size_t kivi_quantized_group_size(const kivi_quantized* q);
size_t kivi_quantized_num_tokens(const kivi_quantized* q);
size_t kivi_quantized_code_bytes(const kivi_quantized* q);
size_t kivi_quantized_metadata_bytes(const kivi_quantized* q);

/* Codes in PackedStream order (concatenated streams), the order of the reference's
 * internal Vec<u32>s (src/quant.rs:307-323, 349-375). code_bytes()/4 words. */
kivi_status kivi_quantized_codes(const kivi_quantized* q, uint32_t* out, size_t out_len,
                                 kivi_error* err);
/* QuantizedTensor::pytorch_codes (src/quant.rs:77-112). code_bytes()/4 words. */
kivi_status kivi_quantized_pytorch_codes(const kivi_quantized* q, uint32_t* out, size_t out_len,
                                         kivi_error* err);
/* Same, into a device buffer, enqueued on `stream`: the PyTorch-KIVI layout without a host
   round trip. */
kivi_status kivi_quantized_pytorch_codes_device(const kivi_quantized* q, uint32_t* out,
                                                size_t out_len, void* stream, kivi_error* err);
/* QuantizedTensor::scale_zero (src/quant.rs:116-121). metadata_bytes()/4 floats. */
kivi_status kivi_quantized_scale_zero(const kivi_quantized* q, float* out, size_t out_len,
                                      kivi_error* err);
/* QuantizedTensor::dequantize (src/quant.rs:124-150). batch*heads*tokens*head_dim floats. */
kivi_status kivi_quantized_dequantize(const kivi_quantized* q, float* out, size_t out_len,
                                      kivi_error* err);
/* Same, into a device buffer, enqueued on `stream`. */
kivi_status kivi_quantized_dequantize_device(const kivi_quantized* q, float* out, size_t out_len,
                                             void* stream, kivi_error* err);

/* ---------------------------------------------------------------- misc */

/* Display text of a status with its payload (src/error.rs:47-95). */
const char* kivi_status_name(int32_t code);
/* ABI version (KIVI_ABI_VERSION) of the loaded library. */
int32_t kivi_abi_version(void);
/* Number of usable HIP devices (0 when none); never fails. */
int32_t kivi_device_count(void);

/* ---------------------------------------------------------------- kernel timing
 * Measurement hooks for benchmark harnesses; no counterpart in the reference, whose path
 * runs on the CPU. While enabled, every launch of a timed kernel family is bracketed by a
 * pair of HIP events on its launch stream and the launch's algorithmic bytes are recorded:
 * the packed and fp32 KV bytes plus the query bytes an attention launch must read, the
 * partials read and outputs written by the merge, and the fp32 rows read plus codes and
 * (scale, zero) written by a quantize launch. kivi_timing_read waits for the pending
 * events and returns the totals since the last kivi_timing_enable call. */
typedef enum kivi_kernel_family {
  KIVI_KERNEL_ATTN_PACKED = 0,  /* attention over 64-token chunks with packed keys and values */
  KIVI_KERNEL_ATTN_TAIL = 1,    /* attention over the rest: windows, residuals, suffixes */
  KIVI_KERNEL_ATTN_MERGE = 2,   /* log-sum-exp merge of the split partials */
  KIVI_KERNEL_QUANT_KEYS = 3,   /* per-channel key quantization into the cache */
  KIVI_KERNEL_QUANT_VALUES = 4, /* per-token value quantization into the cache */
  KIVI_KERNEL_ATTN_SHARED = 5,  /* batched sessions: the shared prefix as a GEMM operand */
  KIVI_KERNEL_ATTN_SESSIONS = 6,/* batched sessions: per-session suffix chunks (or whole sessions) */
  KIVI_KERNEL_CODEC_KEYS = 7,   /* standalone quantize_per_channel */
  KIVI_KERNEL_CODEC_VALUES = 8, /* standalone quantize_per_token */
  KIVI_KERNEL_FAMILIES = 9
} kivi_kernel_family;

typedef struct kivi_kernel_timing {
  uint64_t launches;
  double total_ms;  /* sum of launch durations */
  double bytes;     /* sum of algorithmic bytes */
} kivi_kernel_timing;

/* Enable (non-zero) or disable timing; either way the totals are reset. */
void kivi_timing_enable(int32_t enable);
/* Totals of one kernel family (kivi_kernel_family). */
kivi_status kivi_timing_read(int32_t family, kivi_kernel_timing* out, kivi_error* err);

#ifdef __cplusplus
}
#endif

#endif /* KIVI_AMD_H */
