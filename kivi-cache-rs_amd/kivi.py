"""Python binding over the C ABI in include/kivi.h (ctypes, no compiled glue).

It mirrors the reference crate's public API (bieli/kivi-cache-rs, src/lib.rs:49-64):
``KiviConfig``, ``KiviCache``, ``SharedPrefix``, ``RagSession``, ``RuntimeKv``,
``quantize_per_channel`` / ``quantize_per_token`` -> ``QuantizedTensor`` and
``KiviError``. Arguments mean what they mean in the Rust API; Rust ``&[f32]`` slices
become numpy float32 arrays (any array-like is converted), and ``Result::Err`` becomes
a raised ``KiviError`` carrying the variant name and payload.

Two libraries expose this ABI:
  * ``libkivi_amd.so`` (this package, HIP kernels on the GPU) — ``Backend.amd()``;
  * ``oracle/libkivi_oracle.so`` (CPU restatement of the reference, test-only) —
    loaded by the tests through ``Backend.load(path, prefix="kivi_oracle_")``.
Every object takes the backend it runs on, so a test drives both with the same calls.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "lib" / "libkivi_amd.so"

# ------------------------------------------------------------------ C structs


class _Error(C.Structure):
    _fields_ = [
        ("code", C.c_int32),
        ("a", C.c_uint64),
        ("b", C.c_uint64),
        ("name", C.c_char * 32),
        ("message", C.c_char * 192),
    ]


class _Config(C.Structure):
    _fields_ = [("bits", C.c_uint8), ("group_size", C.c_size_t), ("residual_length", C.c_size_t)]


class _MemoryReport(C.Structure):
    _fields_ = [
        (n, C.c_size_t)
        for n in (
            "tokens",
            "key_code_bytes",
            "key_metadata_bytes",
            "value_code_bytes",
            "value_metadata_bytes",
            "key_residual_bytes",
            "value_residual_bytes",
            "residual_capacity_bytes",
            "fp16_baseline_bytes",
            "fp32_baseline_bytes",
        )
    ]


class _KernelTiming(C.Structure):
    _fields_ = [("launches", C.c_uint64), ("total_ms", C.c_double), ("bytes", C.c_double)]


class _Footprint(C.Structure):
    _fields_ = [
        (n, C.c_size_t)
        for n in (
            "prefix_tokens",
            "question_tokens",
            "sessions",
            "prefix_bytes",
            "question_bytes",
            "shared_total_bytes",
            "fp16_per_user_bytes",
            "fp16_all_users_bytes",
        )
    ]


class _Upgrade(C.Structure):
    _fields_ = [("kind", C.c_uint32), ("from_", C.c_size_t), ("to", C.c_size_t)]


MAX_UPGRADES = 64  # KIVI_MAX_UPGRADES


class _FlushCheck(C.Structure):
    _fields_ = [
        ("sequence_tokens", C.c_size_t),
        ("cosine_before", C.c_float),
        ("cosine", C.c_float),
        ("num_upgrades", C.c_size_t),
        ("upgrades", _Upgrade * MAX_UPGRADES),
    ]


# Variant names of KiviError (reference src/error.rs:5-45) by status code.
VARIANTS = {
    1: "InvalidBits",
    2: "MisalignedGroup",
    3: "ResidualLength",
    4: "HeadDim",
    5: "TokenGroup",
    6: "ZeroDimension",
    7: "Shape",
    8: "QueryHeads",
    9: "EarlyLayers",
    100: "NullArgument",
    101: "Device",
    102: "Capacity",
    103: "Unsupported",
    104: "MismatchedPrefix",
}

# Payload field names per variant, in declaration order (src/error.rs:5-45).
FIELDS = {
    "InvalidBits": ("bits",),
    "MisalignedGroup": ("group_size", "bits"),
    "ResidualLength": ("residual_length", "group_size"),
    "HeadDim": ("head_dim", "group_size"),
    "TokenGroup": ("tokens", "group_size"),
    "Shape": ("expected", "actual"),
    "QueryHeads": ("num_q_heads", "num_kv_heads"),
}


class KiviError(Exception):
    """A ``KiviError`` variant (src/error.rs:5-45) raised from a failed C call."""

    def __init__(self, code: int, a: int, b: int, name: str, message: str):
        super().__init__(message)
        self.code = code
        self.variant = VARIANTS.get(code, f"Unknown{code}")
        self.name = name
        self.message = message
        self.a, self.b = a, b  # raw payload fields of the C status
        self.payload = {}
        for field, value in zip(FIELDS.get(self.variant, ()), (a, b)):
            self.payload[field] = value
        if self.variant == "ZeroDimension":
            self.payload["name"] = name

    def __eq__(self, other):
        if not isinstance(other, KiviError):
            return NotImplemented
        return (self.variant, self.payload) == (other.variant, other.payload)

    def __hash__(self):
        return hash((self.variant, tuple(sorted(self.payload.items()))))

    def __repr__(self):
        fields = ", ".join(f"{k}: {v}" for k, v in self.payload.items())
        return f"KiviError::{self.variant}{{{fields}}}"


# ------------------------------------------------------------------ library


_P = C.c_void_p
_SZ = C.c_size_t
_F32P = C.POINTER(C.c_float)
_U32P = C.POINTER(C.c_uint32)
_ERRP = C.POINTER(_Error)

# name -> (restype, argtypes). Identical for the product and the oracle.
_SIGS = {
    "config_default": (None, [C.POINTER(_Config)]),
    "config_try_new": (C.c_int, [C.c_uint8, _SZ, _SZ, C.POINTER(_Config), _ERRP]),
    "memory_compressed_bytes": (_SZ, [C.POINTER(_MemoryReport)]),
    "memory_compression_ratio_vs_fp16": (C.c_double, [C.POINTER(_MemoryReport)]),
    "footprint_savings_vs_fp16": (C.c_double, [C.POINTER(_Footprint)]),
    "cache_new": (C.c_int, [C.POINTER(_Config), _SZ, _SZ, _SZ, C.POINTER(_P), _ERRP]),
    "cache_free": (None, [_P]),
    "cache_config": (_Config, [_P]),
    "cache_batch_size": (_SZ, [_P]),
    "cache_num_kv_heads": (_SZ, [_P]),
    "cache_head_dim": (_SZ, [_P]),
    "cache_sequence_length": (_SZ, [_P]),
    "cache_key_residual_len": (_SZ, [_P]),
    "cache_value_residual_len": (_SZ, [_P]),
    "cache_quantized_key_tokens": (_SZ, [_P]),
    "cache_quantized_value_tokens": (_SZ, [_P]),
    "cache_tokens_until_key_flush": (_SZ, [_P]),
    "cache_value_residual_slots_remaining": (_SZ, [_P]),
    "cache_append": (C.c_int, [_P, _F32P, _SZ, _F32P, _SZ, _SZ, _ERRP]),
    "cache_attention": (C.c_int, [_P, _F32P, _SZ, _SZ, C.c_float, _F32P, _SZ, _ERRP]),
    "cache_dequantize": (C.c_int, [_P, _F32P, _SZ, _F32P, _SZ, _ERRP]),
    "cache_memory": (_MemoryReport, [_P]),
    "cache_export_streams": (
        C.c_int,
        [_P, _U32P, _SZ, _F32P, _SZ, _U32P, _SZ, _F32P, _SZ, _ERRP],
    ),
    "cache_reserve": (C.c_int, [_P, _SZ, _ERRP]),
    "cache_share_prefix": (C.c_int, [_P, C.POINTER(_P), _ERRP]),
    "prefix_retain": (_P, [_P]),
    "prefix_release": (None, [_P]),
    "prefix_config": (_Config, [_P]),
    "prefix_batch_size": (_SZ, [_P]),
    "prefix_num_kv_heads": (_SZ, [_P]),
    "prefix_head_dim": (_SZ, [_P]),
    "prefix_prefix_tokens": (_SZ, [_P]),
    "prefix_prefix_bytes": (_SZ, [_P]),
    "prefix_shares_allocation_with": (C.c_int, [_P, _P]),
    "prefix_footprint_of": (_Footprint, [_P, _SZ, _SZ]),
    "prefix_session": (C.c_int, [_P, C.POINTER(_P), _ERRP]),
    "session_free": (None, [_P]),
    "session_prefix": (_P, [_P]),
    "session_prefix_tokens": (_SZ, [_P]),
    "session_question_tokens": (_SZ, [_P]),
    "session_sequence_length": (_SZ, [_P]),
    "session_append": (C.c_int, [_P, _F32P, _SZ, _F32P, _SZ, _SZ, _ERRP]),
    "session_attention": (C.c_int, [_P, _F32P, _SZ, _SZ, C.c_float, _F32P, _SZ, _ERRP]),
    "sessions_attention": (
        C.c_int,
        [C.POINTER(_P), _SZ, _F32P, _SZ, _SZ, C.c_float, _F32P, _SZ, _ERRP],
    ),
    "runtime_new": (C.c_int, [C.POINTER(_Config), _SZ, _SZ, _SZ, C.POINTER(_P), _ERRP]),
    "runtime_free": (None, [_P]),
    "runtime_cache": (_P, [_P]),
    "runtime_prefill": (C.c_int, [_P, _F32P, _SZ, _F32P, _SZ, _SZ, _ERRP]),
    "runtime_decode": (
        C.c_int,
        [_P, _F32P, _SZ, _F32P, _SZ, _F32P, _SZ, _SZ, C.c_float, _F32P, _SZ, _ERRP],
    ),
    "guard_new": (
        C.c_int,
        [C.POINTER(_Config), _SZ, _SZ, _SZ, C.c_float, C.c_uint32, C.c_uint8, _SZ,
         C.POINTER(_P), _ERRP],
    ),
    "guard_free": (None, [_P]),
    "guard_config": (_Config, [_P]),
    "guard_cache": (_P, [_P]),
    "guard_policy": (C.c_uint32, [_P]),
    "guard_sequence_length": (_SZ, [_P]),
    "guard_append": (
        C.c_int,
        [_P, _F32P, _SZ, _F32P, _SZ, _SZ, _F32P, _SZ, _SZ, C.c_float,
         C.POINTER(_FlushCheck), _SZ, C.POINTER(_SZ), _ERRP],
    ),
    "guard_last_checks": (_SZ, [_P, _SZ, C.POINTER(_FlushCheck), _SZ]),
    "quantize_per_channel": (
        C.c_int,
        [_F32P, _SZ, _SZ, _SZ, _SZ, _SZ, C.c_uint8, _SZ, C.POINTER(_P), _ERRP],
    ),
    "quantize_per_token": (
        C.c_int,
        [_F32P, _SZ, _SZ, _SZ, _SZ, _SZ, C.c_uint8, _SZ, C.POINTER(_P), _ERRP],
    ),
    "quantized_free": (None, [_P]),
    "quantized_axis": (C.c_int, [_P]),
    "quantized_bits": (C.c_uint8, [_P]),
    "quantized_group_size": (_SZ, [_P]),
    "quantized_num_tokens": (_SZ, [_P]),
    "quantized_code_bytes": (_SZ, [_P]),
    "quantized_metadata_bytes": (_SZ, [_P]),
    "quantized_codes": (C.c_int, [_P, _U32P, _SZ, _ERRP]),
    "quantized_pytorch_codes": (C.c_int, [_P, _U32P, _SZ, _ERRP]),
    "quantized_scale_zero": (C.c_int, [_P, _F32P, _SZ, _ERRP]),
    "quantized_dequantize": (C.c_int, [_P, _F32P, _SZ, _ERRP]),
    "abi_version": (C.c_int32, []),
}

# Entry points only the HIP library has (device pointers, streams, device queries).
_DEVICE_SIGS = {
    "device_count": (C.c_int32, []),
    "timing_enable": (None, [C.c_int32]),
    "timing_read": (C.c_int, [C.c_int32, C.POINTER(_KernelTiming), _ERRP]),
    "status_name": (C.c_char_p, [C.c_int32]),
    "cache_set_stream": (C.c_int, [_P, _P, _ERRP]),
    "cache_append_device": (C.c_int, [_P, _P, _SZ, _P, _SZ, _SZ, _P, _ERRP]),
    "cache_attention_device": (C.c_int, [_P, _P, _SZ, _SZ, C.c_float, _P, _SZ, _P, _ERRP]),
    "cache_attention_device_noalloc": (C.c_int, [_P, _P, _SZ, _SZ, C.c_float, _P, _SZ, _P, _ERRP]),
    "session_append_device": (C.c_int, [_P, _P, _SZ, _P, _SZ, _SZ, _P, _ERRP]),
    "sessions_attention_device": (
        C.c_int,
        [C.POINTER(_P), _SZ, _P, _SZ, _SZ, C.c_float, _P, _SZ, _P, _ERRP],
    ),
    "runtime_decode_device": (
        C.c_int,
        [_P, _P, _SZ, _P, _SZ, _P, _SZ, _SZ, C.c_float, _P, _SZ, _P, _ERRP],
    ),
    "cache_dequantize_device": (C.c_int, [_P, _P, _SZ, _P, _SZ, _P, _ERRP]),
    "cache_export_streams_device": (
        C.c_int,
        [_P, _P, _SZ, _P, _SZ, _P, _SZ, _P, _SZ, _P, _ERRP],
    ),
    "cache_device_bytes": (_SZ, [_P]),
    "plan_device_bytes": (C.c_int, [C.POINTER(_Config), _SZ, _SZ, _SZ, _SZ, C.POINTER(_SZ), _ERRP]),
    "quantized_pytorch_codes_device": (C.c_int, [_P, _P, _SZ, _P, _ERRP]),
    "quantized_dequantize_device": (C.c_int, [_P, _P, _SZ, _P, _ERRP]),
    "quantize_per_channel_device": (
        C.c_int,
        [_P, _SZ, _SZ, _SZ, _SZ, _SZ, C.c_uint8, _SZ, _P, C.POINTER(_P), _ERRP],
    ),
    "quantize_per_token_device": (
        C.c_int,
        [_P, _SZ, _SZ, _SZ, _SZ, _SZ, C.c_uint8, _SZ, _P, C.POINTER(_P), _ERRP],
    ),
}


class Backend:
    """One loaded library exposing the kivi C ABI under ``prefix``."""

    _cache: dict = {}

    def __init__(self, path, prefix="kivi_", device=True):
        self.path = str(path)
        self.prefix = prefix
        self.lib = C.CDLL(self.path)
        self.device = device
        sigs = dict(_SIGS)
        if device:
            sigs.update(_DEVICE_SIGS)
        self.fn = {}
        for name, (res, args) in sigs.items():
            f = getattr(self.lib, prefix + name)
            f.restype = res
            f.argtypes = args
            self.fn[name] = f

    @classmethod
    def load(cls, path, prefix="kivi_", device=True):
        key = (str(path), prefix)
        if key not in cls._cache:
            cls._cache[key] = cls(path, prefix, device)
        return cls._cache[key]

    @classmethod
    def amd(cls):
        """The HIP library built in-tree (``kivi-cache-rs_amd/lib/libkivi_amd.so``)."""
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built; run __graft_entry__.build() (make -C kivi-cache-rs_amd)"
            )
        return cls.load(LIB_PATH, "kivi_", True)

    def call(self, name, *args):
        err = _Error()
        rc = self.fn[name](*args, C.byref(err))
        if rc != 0:
            raise KiviError(
                err.code, err.a, err.b, err.name.decode(errors="replace"),
                err.message.decode(errors="replace"),
            )

    def __getitem__(self, name):
        return self.fn[name]


# ------------------------------------------------------------------ helpers


def _f32(x):
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32)).reshape(-1)
    return a


def _fptr(a):
    return a.ctypes.data_as(_F32P) if a.size else None


def _uptr(a):
    return a.ctypes.data_as(_U32P) if a.size else None


class KiviConfig:
    """``KiviConfig`` (src/config.rs:9-45)."""

    __slots__ = ("bits", "group_size", "residual_length")

    def __init__(self, bits=2, group_size=32, residual_length=128):
        self.bits, self.group_size, self.residual_length = bits, group_size, residual_length

    @classmethod
    def default(cls):
        return cls()

    @classmethod
    def try_new(cls, backend, bits, group_size, residual_length):
        out = _Config()
        backend.call("config_try_new", bits, group_size, residual_length, C.byref(out))
        return cls(out.bits, out.group_size, out.residual_length)

    def _c(self):
        return _Config(self.bits, self.group_size, self.residual_length)

    def __eq__(self, other):
        return (self.bits, self.group_size, self.residual_length) == (
            other.bits, other.group_size, other.residual_length)

    def __repr__(self):
        return f"KiviConfig(bits={self.bits}, group_size={self.group_size}, residual_length={self.residual_length})"


class MemoryReport:
    """``MemoryReport`` (src/cache.rs:25-58)."""

    def __init__(self, backend, raw):
        self._b, self._raw = backend, raw
        for name, _ in _MemoryReport._fields_:
            setattr(self, name, getattr(raw, name))

    def compressed_bytes(self):
        return self._b["memory_compressed_bytes"](C.byref(self._raw))

    def compression_ratio_vs_fp16(self):
        return self._b["memory_compression_ratio_vs_fp16"](C.byref(self._raw))


class SharedPrefixFootprint:
    """``SharedPrefixFootprint`` (src/prefix.rs:51-71)."""

    def __init__(self, backend, raw):
        self._b, self._raw = backend, raw
        for name, _ in _Footprint._fields_:
            setattr(self, name, getattr(raw, name))

    def savings_vs_fp16(self):
        return self._b["footprint_savings_vs_fp16"](C.byref(self._raw))


class KiviCache:
    """``KiviCache`` (src/cache.rs:71-380) over the backend's C ABI."""

    def __init__(self, backend, config, batch, num_kv_heads, head_dim, _handle=None, _owner=True):
        self._b = backend
        self._owner = _owner
        if _handle is not None:
            self._h = _handle
            return
        h = C.c_void_p()
        backend.call("cache_new", C.byref(config._c()), batch, num_kv_heads, head_dim, C.byref(h))
        self._h = h

    @classmethod
    def new(cls, backend, config, batch, num_kv_heads, head_dim):
        return cls(backend, config, batch, num_kv_heads, head_dim)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h and self._owner:
            self._b["cache_free"](h)
            self._h = None

    # getters (src/cache.rs:122-156, 328-337)
    def config(self):
        c = self._b["cache_config"](self._h)
        return KiviConfig(c.bits, c.group_size, c.residual_length)

    def batch_size(self):
        return self._b["cache_batch_size"](self._h)

    def num_kv_heads(self):
        return self._b["cache_num_kv_heads"](self._h)

    def head_dim(self):
        return self._b["cache_head_dim"](self._h)

    def sequence_length(self):
        return self._b["cache_sequence_length"](self._h)

    def key_residual_len(self):
        return self._b["cache_key_residual_len"](self._h)

    def value_residual_len(self):
        return self._b["cache_value_residual_len"](self._h)

    def quantized_key_tokens(self):
        return self._b["cache_quantized_key_tokens"](self._h)

    def quantized_value_tokens(self):
        return self._b["cache_quantized_value_tokens"](self._h)

    def tokens_until_key_flush(self):
        return self._b["cache_tokens_until_key_flush"](self._h)

    def value_residual_slots_remaining(self):
        return self._b["cache_value_residual_slots_remaining"](self._h)

    def append(self, keys, values, seq_len):
        k, v = _f32(keys), _f32(values)
        self._b.call("cache_append", self._h, _fptr(k), k.size, _fptr(v), v.size, seq_len)

    def attention(self, query, num_q_heads, scale):
        q = _f32(query)
        n = self.batch_size() * num_q_heads * self.head_dim()
        out = np.zeros(max(n, 0), dtype=np.float32)
        self._b.call("cache_attention", self._h, _fptr(q), q.size, num_q_heads,
                     C.c_float(scale), _fptr(out), out.size)
        return out

    def dequantize(self):
        n = self.batch_size() * self.num_kv_heads() * self.sequence_length() * self.head_dim()
        k = np.zeros(n, dtype=np.float32)
        v = np.zeros(n, dtype=np.float32)
        self._b.call("cache_dequantize", self._h, _fptr(k), k.size, _fptr(v), v.size)
        return k, v

    def memory(self):
        return MemoryReport(self._b, self._b["cache_memory"](self._h))

    def stream_lengths(self):
        cfg = self.config()
        units = self.batch_size() * self.num_kv_heads()
        d = self.head_dim()
        kq, vq = self.quantized_key_tokens(), self.quantized_value_tokens()
        return (
            units * kq * d * cfg.bits // 32,
            units * 2 * (kq // cfg.group_size) * d,
            units * vq * d * cfg.bits // 32,
            units * 2 * vq * (d // cfg.group_size),
        )

    def export_streams(self):
        """Packed streams in the reference PackedStream order (src/quant.rs:37-44)."""
        nkc, nkp, nvc, nvp = self.stream_lengths()
        kc = np.zeros(nkc, dtype=np.uint32)
        kp = np.zeros(nkp, dtype=np.float32)
        vc = np.zeros(nvc, dtype=np.uint32)
        vp = np.zeros(nvp, dtype=np.float32)
        self._b.call("cache_export_streams", self._h, _uptr(kc), nkc, _fptr(kp), nkp,
                     _uptr(vc), nvc, _fptr(vp), nvp)
        return kc, kp, vc, vp

    def reserve(self, tokens):
        self._b.call("cache_reserve", self._h, tokens)

    def share_prefix(self):
        h = C.c_void_p()
        self._b.call("cache_share_prefix", self._h, C.byref(h))
        return SharedPrefix(self._b, h)

    # device entry points (HIP library only)
    def set_stream(self, stream_ptr):
        self._b.call("cache_set_stream", self._h, C.c_void_p(stream_ptr))

    def append_device(self, k_ptr, k_len, v_ptr, v_len, seq_len, stream=0):
        self._b.call("cache_append_device", self._h, C.c_void_p(k_ptr), k_len,
                     C.c_void_p(v_ptr), v_len, seq_len, C.c_void_p(stream))

    def attention_device(self, q_ptr, q_len, num_q_heads, scale, out_ptr, out_len, stream=0):
        self._b.call("cache_attention_device", self._h, C.c_void_p(q_ptr), q_len, num_q_heads,
                     C.c_float(scale), C.c_void_p(out_ptr), out_len, C.c_void_p(stream))

    def attention_device_noalloc(self, q_ptr, q_len, num_q_heads, scale, out_ptr, out_len, stream=0):
        """attention_device with the split partials in the library's static per-device
        workspace (no allocation; see kivi_cache_attention_device_noalloc)."""
        self._b.call("cache_attention_device_noalloc", self._h, C.c_void_p(q_ptr), q_len, num_q_heads,
                     C.c_float(scale), C.c_void_p(out_ptr), out_len, C.c_void_p(stream))

    def dequantize_device(self, k_ptr, k_len, v_ptr, v_len, stream=0):
        self._b.call("cache_dequantize_device", self._h, C.c_void_p(k_ptr), k_len,
                     C.c_void_p(v_ptr), v_len, C.c_void_p(stream))

    def export_streams_device(self, ptrs, lens, stream=0):
        """``ptrs``/``lens``: key codes, key params, value codes, value params (0 = skip)."""
        args = []
        for p, n in zip(ptrs, lens):
            args += [C.c_void_p(p or None), n]
        self._b.call("cache_export_streams_device", self._h, *args, C.c_void_p(stream))

    def device_bytes(self):
        return self._b["cache_device_bytes"](self._h)


class SharedPrefix:
    """``SharedPrefix`` (src/prefix.rs:29-153); the handle holds one reference."""

    def __init__(self, backend, handle):
        self._b, self._h = backend, handle

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._b["prefix_release"](h)
            self._h = None

    def clone(self):
        return SharedPrefix(self._b, C.c_void_p(self._b["prefix_retain"](self._h)))

    def config(self):
        c = self._b["prefix_config"](self._h)
        return KiviConfig(c.bits, c.group_size, c.residual_length)

    def batch_size(self):
        return self._b["prefix_batch_size"](self._h)

    def num_kv_heads(self):
        return self._b["prefix_num_kv_heads"](self._h)

    def head_dim(self):
        return self._b["prefix_head_dim"](self._h)

    def prefix_tokens(self):
        return self._b["prefix_prefix_tokens"](self._h)

    def prefix_bytes(self):
        return self._b["prefix_prefix_bytes"](self._h)

    def shares_allocation_with(self, other):
        return bool(self._b["prefix_shares_allocation_with"](self._h, other._h))

    def footprint(self, sessions, question_tokens):
        return SharedPrefixFootprint(
            self._b, self._b["prefix_footprint_of"](self._h, sessions, question_tokens))

    def session(self):
        h = C.c_void_p()
        self._b.call("prefix_session", self._h, C.byref(h))
        return RagSession(self._b, h, self)


class RagSession:
    """``RagSession`` (src/prefix.rs:41-46, 155-289)."""

    def __init__(self, backend, handle, parent):
        self._b, self._h = backend, handle
        self._parent = parent  # keeps the Python prefix alive for prefix()

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._b["session_free"](h)
            self._h = None

    def prefix(self):
        view = SharedPrefix(self._b, C.c_void_p(self._b["prefix_retain"](
            C.c_void_p(self._b["session_prefix"](self._h)))))
        return view

    def prefix_tokens(self):
        return self._b["session_prefix_tokens"](self._h)

    def question_tokens(self):
        return self._b["session_question_tokens"](self._h)

    def sequence_length(self):
        return self._b["session_sequence_length"](self._h)

    def append(self, keys, values, seq_len):
        k, v = _f32(keys), _f32(values)
        self._b.call("session_append", self._h, _fptr(k), k.size, _fptr(v), v.size, seq_len)

    def attention(self, query, num_q_heads, scale):
        q = _f32(query)
        p = self._parent
        n = p.batch_size() * num_q_heads * p.head_dim()
        out = np.zeros(max(n, 0), dtype=np.float32)
        self._b.call("session_attention", self._h, _fptr(q), q.size, num_q_heads,
                     C.c_float(scale), _fptr(out), out.size)
        return out

    def append_device(self, k_ptr, k_len, v_ptr, v_len, seq_len, stream=0):
        self._b.call("session_append_device", self._h, C.c_void_p(k_ptr), k_len,
                     C.c_void_p(v_ptr), v_len, seq_len, C.c_void_p(stream))


# kivi_kernel_family (include/kivi.h)
KERNEL_FAMILIES = {"attn_packed": 0, "attn_tail": 1, "attn_merge": 2, "quant_keys": 3,
                   "quant_values": 4, "attn_shared": 5, "attn_sessions": 6, "codec_keys": 7,
                   "codec_values": 8}


def timing_enable(backend, on=True):
    """Start (or stop) per-launch HIP-event timing of the library's kernels; resets totals."""
    backend["timing_enable"](1 if on else 0)


def timing_read(backend, family):
    """(launches, total_ms, algorithmic bytes) of one kernel family since timing_enable."""
    t = _KernelTiming()
    backend.call("timing_read", KERNEL_FAMILIES[family] if isinstance(family, str) else family,
                 C.byref(t))
    return t.launches, t.total_ms, t.bytes


def sessions_attention(backend, sessions, queries, num_q_heads, scale):
    """Batched ``RagSession::attention`` over sessions of one prefix (C-ABI extension)."""
    q = _f32(queries)
    n = len(sessions)
    arr = session_handles(sessions)
    if n:
        p = sessions[0]._parent
        per = p.batch_size() * num_q_heads * p.head_dim()
    else:
        per = 0
    out = np.zeros(n * per, dtype=np.float32)
    backend.call("sessions_attention", C.cast(arr, C.POINTER(C.c_void_p)), n, _fptr(q), q.size,
                 num_q_heads, C.c_float(scale), _fptr(out), out.size)
    return out


def session_handles(sessions):
    """ctypes array of the sessions' handles (the ``const kivi_session* const*`` argument)."""
    return (C.c_void_p * max(len(sessions), 1))(
        *[s._h.value if isinstance(s._h, C.c_void_p) else s._h for s in sessions])


def sessions_attention_device(backend, sessions, q_ptr, q_len, num_q_heads, scale, out_ptr,
                              out_len, stream=0, handles=None):
    """Device-pointer form of :func:`sessions_attention`, enqueued on ``stream``. ``handles``
    (from :func:`session_handles`) skips rebuilding the handle array on every call."""
    arr = session_handles(sessions) if handles is None else handles
    backend.call("sessions_attention_device", C.cast(arr, C.POINTER(C.c_void_p)), len(sessions),
                 C.c_void_p(q_ptr), q_len, num_q_heads, C.c_float(scale), C.c_void_p(out_ptr),
                 out_len, C.c_void_p(stream))
    return arr


class RuntimeKv:
    """``RuntimeKv`` (src/runtime.rs:12-57)."""

    def __init__(self, backend, config, batch, num_kv_heads, head_dim):
        self._b = backend
        h = C.c_void_p()
        backend.call("runtime_new", C.byref(config._c()), batch, num_kv_heads, head_dim,
                     C.byref(h))
        self._h = h

    @classmethod
    def try_new(cls, backend, config, batch, num_kv_heads, head_dim):
        return cls(backend, config, batch, num_kv_heads, head_dim)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._b["runtime_free"](h)
            self._h = None

    def cache(self):
        ch = C.c_void_p(self._b["runtime_cache"](self._h))
        c = KiviCache(self._b, None, 0, 0, 0, _handle=ch, _owner=False)
        c._rt = self  # keep the runtime alive while the borrowed cache is used
        return c

    def prefill(self, keys, values, seq_len):
        k, v = _f32(keys), _f32(values)
        self._b.call("runtime_prefill", self._h, _fptr(k), k.size, _fptr(v), v.size, seq_len)

    def decode(self, key, value, query, num_q_heads, scale):
        k, v, q = _f32(key), _f32(value), _f32(query)
        c = self.cache()
        n = c.batch_size() * num_q_heads * c.head_dim()
        out = np.zeros(max(n, 0), dtype=np.float32)
        self._b.call("runtime_decode", self._h, _fptr(k), k.size, _fptr(v), v.size, _fptr(q),
                     q.size, num_q_heads, C.c_float(scale), _fptr(out), out.size)
        return out

    def decode_device(self, k_ptr, k_len, v_ptr, v_len, q_ptr, q_len, num_q_heads, scale, out_ptr,
                      out_len, stream=0):
        self._b.call("runtime_decode_device", self._h, C.c_void_p(k_ptr), k_len, C.c_void_p(v_ptr),
                     v_len, C.c_void_p(q_ptr), q_len, num_q_heads, C.c_float(scale),
                     C.c_void_p(out_ptr), out_len, C.c_void_p(stream))


class QualityPolicy:
    """``QualityPolicy`` (src/guard.rs:13-19)."""

    RaiseBits = 0
    LengthenResidual = 1


class QualityUpgrade:
    """``QualityUpgrade`` (src/guard.rs:22-26): ``kind`` is "Bits" or "Residual"."""

    __slots__ = ("kind", "from_", "to")

    def __init__(self, kind, from_, to):
        self.kind, self.from_, self.to = kind, from_, to

    @classmethod
    def bits(cls, from_, to):
        return cls("Bits", from_, to)

    @classmethod
    def residual(cls, from_, to):
        return cls("Residual", from_, to)

    def __eq__(self, other):
        return isinstance(other, QualityUpgrade) and (self.kind, self.from_, self.to) == (
            other.kind, other.from_, other.to)

    def __repr__(self):
        return f"{self.kind} {{ from: {self.from_}, to: {self.to} }}"


class FlushCheck:
    """``FlushCheck`` (src/guard.rs:29-35)."""

    __slots__ = ("sequence_tokens", "cosine_before", "cosine", "upgrades")

    def __init__(self, raw):
        self.sequence_tokens = raw.sequence_tokens
        self.cosine_before = raw.cosine_before
        self.cosine = raw.cosine
        self.upgrades = [
            QualityUpgrade("Bits" if u.kind == 0 else "Residual", u.from_, u.to)
            for u in raw.upgrades[: raw.num_upgrades]
        ]

    def __repr__(self):
        return (f"FlushCheck(sequence_tokens={self.sequence_tokens}, "
                f"cosine_before={self.cosine_before}, cosine={self.cosine}, "
                f"upgrades={self.upgrades})")


class QualityGuard:
    """``QualityGuard`` (src/guard.rs:37-258): a cache plus the fp32 tape of its tokens; after
    each key flush cache attention is scored against fp32 attention (cosine) and the cache is
    rebuilt with wider codes or a longer residual window while the score misses ``threshold``."""

    def __init__(self, backend, config, batch, num_kv_heads, head_dim, threshold, policy,
                 max_bits, max_residual):
        self._b = backend
        h = C.c_void_p()
        backend.call("guard_new", C.byref(config._c()), batch, num_kv_heads, head_dim,
                     C.c_float(threshold), policy, max_bits, max_residual, C.byref(h))
        self._h = h

    @classmethod
    def try_new(cls, backend, config, batch, num_kv_heads, head_dim, threshold, policy, max_bits,
                max_residual):
        return cls(backend, config, batch, num_kv_heads, head_dim, threshold, policy, max_bits,
                   max_residual)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._b["guard_free"](h)
            self._h = None

    def config(self):
        c = self._b["guard_config"](self._h)
        return KiviConfig(c.bits, c.group_size, c.residual_length)

    def cache(self):
        """The resident cache, borrowed: valid until the next append that upgrades."""
        ch = C.c_void_p(self._b["guard_cache"](self._h))
        c = KiviCache(self._b, None, 0, 0, 0, _handle=ch, _owner=False)
        c._guard = self
        return c

    def policy(self):
        return self._b["guard_policy"](self._h)

    def sequence_length(self):
        return self._b["guard_sequence_length"](self._h)

    def append(self, keys, values, seq_len, query, num_q_heads, scale):
        k, v, q = _f32(keys), _f32(values), _f32(query)
        cap = 8
        buf = (_FlushCheck * cap)()
        n = _SZ(0)
        self._b.call("guard_append", self._h, _fptr(k), k.size, _fptr(v), v.size, seq_len,
                     _fptr(q), q.size, num_q_heads, C.c_float(scale), buf, cap, C.byref(n))
        if n.value > cap:
            buf = (_FlushCheck * n.value)()
            got = self._b["guard_last_checks"](self._h, 0, buf, n.value)
            assert got == n.value
        return [FlushCheck(buf[i]) for i in range(n.value)]


PER_CHANNEL, PER_TOKEN = 0, 1


class QuantizedTensor:
    """``QuantizedTensor`` (src/quant.rs:24-151)."""

    def __init__(self, backend, handle, shape):
        self._b, self._h = backend, handle
        self.batch, self.heads, self.tokens, self.head_dim = shape

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._b["quantized_free"](h)
            self._h = None

    def axis(self):
        return self._b["quantized_axis"](self._h)

    def bits(self):
        return self._b["quantized_bits"](self._h)

    def group_size(self):
        return self._b["quantized_group_size"](self._h)

    def num_tokens(self):
        return self._b["quantized_num_tokens"](self._h)

    def code_bytes(self):
        return self._b["quantized_code_bytes"](self._h)

    def metadata_bytes(self):
        return self._b["quantized_metadata_bytes"](self._h)

    def codes(self):
        out = np.zeros(self.code_bytes() // 4, dtype=np.uint32)
        self._b.call("quantized_codes", self._h, _uptr(out), out.size)
        return out

    def pytorch_codes(self):
        out = np.zeros(self.code_bytes() // 4, dtype=np.uint32)
        self._b.call("quantized_pytorch_codes", self._h, _uptr(out), out.size)
        return out

    def scale_zero(self):
        out = np.zeros(self.metadata_bytes() // 4, dtype=np.float32)
        self._b.call("quantized_scale_zero", self._h, _fptr(out), out.size)
        return out

    def dequantize(self):
        out = np.zeros(self.batch * self.heads * self.tokens * self.head_dim, dtype=np.float32)
        self._b.call("quantized_dequantize", self._h, _fptr(out), out.size)
        return out

    def pytorch_codes_device(self, out_ptr, out_len, stream=0):
        self._b.call("quantized_pytorch_codes_device", self._h, C.c_void_p(out_ptr), out_len,
                     C.c_void_p(stream))

    def dequantize_device(self, out_ptr, out_len, stream=0):
        self._b.call("quantized_dequantize_device", self._h, C.c_void_p(out_ptr), out_len,
                     C.c_void_p(stream))


def plan_device_bytes(backend, config, batch, num_kv_heads, head_dim, tokens):
    """HBM a cache of this shape holds after ``reserve(tokens)`` (HIP library only)."""
    out = _SZ(0)
    backend.call("plan_device_bytes", C.byref(config._c()), batch, num_kv_heads, head_dim, tokens,
                 C.byref(out))
    return out.value


def _quantize(backend, name, data, batch, heads, tokens, head_dim, bits, group_size):
    a = _f32(data)
    h = C.c_void_p()
    backend.call(name, _fptr(a), a.size, batch, heads, tokens, head_dim, bits, group_size,
                 C.byref(h))
    return QuantizedTensor(backend, h, (batch, heads, tokens, head_dim))


def quantize_per_channel(backend, data, batch, heads, tokens, head_dim, bits, group_size):
    """``quantize_per_channel`` (src/quant.rs:153-191)."""
    return _quantize(backend, "quantize_per_channel", data, batch, heads, tokens, head_dim, bits,
                     group_size)


def quantize_per_token(backend, data, batch, heads, tokens, head_dim, bits, group_size):
    """``quantize_per_token`` (src/quant.rs:193-233)."""
    return _quantize(backend, "quantize_per_token", data, batch, heads, tokens, head_dim, bits,
                     group_size)


def quantize_device(backend, per_channel, data_ptr, data_len, batch, heads, tokens, head_dim, bits,
                    group_size, stream=0):
    """``quantize_per_channel`` / ``quantize_per_token`` on device input, enqueued on ``stream``
    (HIP library only)."""
    h = C.c_void_p()
    name = "quantize_per_channel_device" if per_channel else "quantize_per_token_device"
    backend.call(name, C.c_void_p(data_ptr), data_len, batch, heads, tokens, head_dim, bits,
                 group_size, C.c_void_p(stream), C.byref(h))
    return QuantizedTensor(backend, h, (batch, heads, tokens, head_dim))


# ------------------------------------------------------------------ seeded inputs


def lcg_fill(n, seed):
    """The reference tests' LCG (tests/attention.rs:3-11): exact in f32 on any IEEE host."""
    out = np.empty(n, dtype=np.float32)
    # state = state*1664525 + 1013904223 (mod 2^32): Python ints for small n, a blocked
    # jump-ahead in numpy for large n.
    if n <= 4096:
        s = int(seed) & 0xFFFFFFFF
        vals = []
        for _ in range(n):
            s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
            vals.append(s >> 8)
        u = np.asarray(vals, dtype=np.float32)
    else:
        u = _lcg_states(seed, n).astype(np.float32)
    u = u / np.float32(1 << 24)
    out[:] = u * np.float32(2.0) - np.float32(1.0)
    return out


def _lcg_states(seed, n):
    """(state >> 8) for the first n LCG steps, computed with a parallel jump-ahead."""
    a, c, m = 1664525, 1013904223, 1 << 32
    block = 4096
    nb = (n + block - 1) // block
    # powers for the first block
    first = np.empty(block, dtype=np.uint64)
    s = int(seed) & 0xFFFFFFFF
    for i in range(block):
        s = (s * a + c) % m
        first[i] = s
    # jump of `block` steps: state' = A*state + Cc (mod m)
    A, Cc = 1, 0
    for _ in range(block):
        A, Cc = (A * a) % m, (Cc * a + c) % m
    states = np.empty((nb, block), dtype=np.uint64)
    states[0] = first
    mask = np.uint64(0xFFFFFFFF)
    A64, C64 = np.uint64(A), np.uint64(Cc)
    for bi in range(1, nb):
        # (A*x + C) mod 2^32 with 64-bit wraparound is exact modulo 2^32
        states[bi] = (states[bi - 1] * A64 + C64) & mask
    return (states.reshape(-1)[:n] >> np.uint64(8))
