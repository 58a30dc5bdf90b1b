"""TEST INFRASTRUCTURE ONLY: ctypes bindings of the C oracle (oracle/kvb_oracle.h, built into
oracle/build/libkvb_oracle.so) and, when it was built, of the reference's own CPU code compiled
into oracle/_ref/libkvbref.so (oracle/Makefile `ref`, from chipontix/kv-cache-bench
src/reference.cpp). Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# KVBO_LIB: a build of a mutated copy of kvb_oracle.c (tests/mutation/mutate.py); unset, the in-tree build
LIB = os.environ.get("KVBO_LIB") or os.path.join(HERE, "build", "libkvb_oracle.so")
REF = os.path.join(HERE, "_ref", "libkvbref.so")

_p, _i, _sz, _dbl = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.c_double


class Shape(ctypes.Structure):
    _fields_ = [("batch", _i), ("num_heads", _i), ("num_kv_heads", _i), ("head_dim", _i)]


_SP = ctypes.POINTER(Shape)

lib = ctypes.CDLL(LIB)
for name, args, ret in [
    ("kvbo_f16_to_f32", [ctypes.c_uint16], ctypes.c_float),
    ("kvbo_f32_to_f16", [ctypes.c_float], ctypes.c_uint16),
    ("kvbo_max_abs_diff", [_p, _p, _sz], _dbl),
    ("kvbo_mt64_seed", [_p, ctypes.c_uint64], None),
    ("kvbo_mt64_next", [_p], ctypes.c_uint64),
    ("kvbo_layout_dims", [_p, _i, _i, _dbl, _p, _p, _p], _i),
    ("kvbo_make_paged_layout", [_p, _i, _i, _dbl, ctypes.c_uint64, _p], _i),
    ("kvbo_scatter_to_paged", [_SP, _i, _i, _p, _p, _i, _sz, _p, _p], None),
    ("kvbo_quantize_to_paged_i8", [_SP, _i, _i, _p, _p, _i, _p, _p, _p], None),
    ("kvbo_dequantize_paged_i8", [_SP, _i, _i, _p, _p, _i, _p, _p, _p], None),
    ("kvbo_attention_f32", [_SP, _p, _i, _p, _p, _p, _p, ctypes.c_float, _i], None),
    ("kvbo_attention_f16", [_SP, _p, _i, _p, _p, _p, _p, ctypes.c_float, _i], None),
    ("kvbo_partition_state_f32", [_SP, _p, _i, _p, _p, _p, ctypes.c_float, _i, _i, _i, _i, _p, _p, _p], _i),
    ("kvbo_auto_part_tokens", [_i, _i, _i], _i),
    ("kvbo_split_decode", [_SP, _i, _i, _i, _p, _p, _i, _p, _p, _p, _p, _p, ctypes.c_float, _i, _i, _p, _p, _p, _i], _i),
    ("kvbo_fp16_storage_bound", [_SP, _p, _i, _p, _p, _p], _dbl),
    ("kvbo_i8_storage_bound", [_SP, _p, _i, _i, _p, _p, _p, _p], _dbl),
]:
    f = getattr(lib, name)
    f.argtypes, f.restype = args, ret

ref = None
if os.path.exists(REF):
    ref = ctypes.CDLL(REF)
    for name, args, ret in [
        ("kvbref_attention_f32", [_i, _i, _i, _i, _p, _i, _p, _p, _p, _p, ctypes.c_float, _i], None),
        ("kvbref_attention_f16", [_i, _i, _i, _i, _p, _i, _p, _p, _p, _p, ctypes.c_float, _i], None),
        ("kvbref_make_paged_layout", [_p, _i, _i, ctypes.c_uint64, _p, _sz, _p], _i),
        ("kvbref_quantize_to_paged_i8", [_i, _i, _i, _i, _i, _i, _i, _p, _p, _i, _p, _p, _p], None),
        ("kvbref_dequantize_paged_i8", [_i, _i, _i, _i, _i, _i, _i, _p, _p, _i, _p, _p, _p], None),
        ("kvbref_scatter_to_paged_f32", [_i, _i, _i, _i, _i, _i, _i, _p, _p, _i, _p, _p], None),
        ("kvbref_max_abs_diff", [_p, _p, _sz], _dbl),
        ("kvbref_auto_part_tokens", [_i, _i, _i, _i, _i], _i),
    ]:
        f = getattr(ref, name)
        f.argtypes, f.restype = args, ret


def _ptr(a):
    return None if a is None else a.ctypes.data_as(_p)


def shape_of(s):
    return Shape(s.batch, s.num_heads, s.num_kv_heads, s.head_dim)


def scale_of(head_dim):
    return float(np.float32(1.0) / np.float32(np.sqrt(np.float32(head_dim))))


def attention(shape, lens, max_len, q, k, v, scale=None, threads=1):
    """fp64 two-pass reference on the contiguous cache; k/v float32 or float16 (stored values)."""
    lens = np.ascontiguousarray(lens, np.int32)
    q = np.ascontiguousarray(q, np.float32)
    out = np.empty((shape.batch, shape.num_heads, shape.head_dim), np.float32)
    sc = scale_of(shape.head_dim) if scale is None else scale
    s = shape_of(shape)
    if k.dtype == np.float16:
        lib.kvbo_attention_f16(ctypes.byref(s), _ptr(lens), max_len, _ptr(q), _ptr(np.ascontiguousarray(k)),
                               _ptr(np.ascontiguousarray(v)), _ptr(out), sc, threads)
    else:
        lib.kvbo_attention_f32(ctypes.byref(s), _ptr(lens), max_len, _ptr(q),
                               _ptr(np.ascontiguousarray(k, np.float32)), _ptr(np.ascontiguousarray(v, np.float32)),
                               _ptr(out), sc, threads)
    return out


def ref_attention(shape, lens, max_len, q, k, v, scale=None, threads=1):
    """The reference's own attention_reference (oracle/_ref), or None if it was not built."""
    if ref is None:
        return None
    lens = np.ascontiguousarray(lens, np.int32)
    q = np.ascontiguousarray(q, np.float32)
    out = np.empty((shape.batch, shape.num_heads, shape.head_dim), np.float32)
    sc = scale_of(shape.head_dim) if scale is None else scale
    fn = ref.kvbref_attention_f16 if k.dtype == np.float16 else ref.kvbref_attention_f32
    fn(shape.batch, shape.num_heads, shape.num_kv_heads, shape.head_dim, _ptr(lens), max_len, _ptr(q),
       _ptr(np.ascontiguousarray(k)), _ptr(np.ascontiguousarray(v)), _ptr(out), sc, threads)
    return out


def partition_state(shape, lens, max_len, q, k, v, part_tokens, b, h, p, scale=None):
    """(m, l, o[D]) of one split-K partition in fp64, or None if it is empty."""
    lens = np.ascontiguousarray(lens, np.int32)
    m, l = ctypes.c_double(), ctypes.c_double()
    o = np.empty(shape.head_dim, np.float64)
    sc = scale_of(shape.head_dim) if scale is None else scale
    s = shape_of(shape)
    wrote = lib.kvbo_partition_state_f32(ctypes.byref(s), _ptr(lens), max_len, _ptr(np.ascontiguousarray(q, np.float32)),
                                         _ptr(np.ascontiguousarray(k, np.float32)),
                                         _ptr(np.ascontiguousarray(v, np.float32)), sc, part_tokens, b, h, p,
                                         ctypes.byref(m), ctypes.byref(l), _ptr(o))
    return (m.value, l.value, o) if wrote else None


KV_KIND = {np.dtype(np.float32): 0, np.dtype(np.float16): 1, np.dtype(np.int8): 2}


def split_decode(shape, page, table, lens, max_len, q, k_pool, v_pool, k_scale=None, v_scale=None, part_tokens=0,
                 waves=None, scale=None, threads=8):
    """The CPU model of the split-K decode kernel over the paged pool (kvbo_split_decode):
    (out [B][H][D], part_out [B][H][max_parts][D], part_ml [B][H][max_parts][2]). The storage type
    comes from the pool's dtype; waves default to the kernel's 4 per workgroup."""
    kind = KV_KIND[np.dtype(k_pool.dtype)]
    waves = 4 if waves is None else waves
    table = np.ascontiguousarray(table, np.int32)
    lens = np.ascontiguousarray(lens, np.int32)
    sc = scale_of(shape.head_dim) if scale is None else scale
    part = part_tokens or auto_part_tokens(shape.batch, shape.num_kv_heads, max_len)
    max_parts = max(1, -(-max_len // part))
    B, H, D = shape.batch, shape.num_heads, shape.head_dim
    out = np.full((B, H, D), np.nan, np.float32)
    part_out = np.empty((B, H, max_parts, D), np.float32)
    part_ml = np.empty((B, H, max_parts, 2), np.float32)
    s = shape_of(shape)
    k_pool, v_pool = np.ascontiguousarray(k_pool), np.ascontiguousarray(v_pool)
    ks = None if k_scale is None else np.ascontiguousarray(k_scale, np.float32)
    vs = None if v_scale is None else np.ascontiguousarray(v_scale, np.float32)
    got = lib.kvbo_split_decode(ctypes.byref(s), kind, page, table.shape[1], _ptr(table), _ptr(lens), max_len,
                                _ptr(np.ascontiguousarray(q, np.float32)), _ptr(k_pool), _ptr(v_pool), _ptr(ks),
                                _ptr(vs), sc, part, waves, _ptr(part_out), _ptr(part_ml), _ptr(out), threads)
    if got != max_parts:
        raise ValueError(f"kvbo_split_decode refused its arguments ({got})")
    return out, part_out, part_ml


def layout_dims(lens, page, pool_factor=1.0):
    lens = np.ascontiguousarray(lens, np.int32)
    mb, live, pool = _i(), _i(), _i()
    rc = lib.kvbo_layout_dims(_ptr(lens), len(lens), page, pool_factor, ctypes.byref(mb), ctypes.byref(live),
                              ctypes.byref(pool))
    if rc:
        raise ValueError("bad layout arguments")
    return mb.value, live.value, pool.value


def make_paged_layout(lens, page, seed, pool_factor=1.0):
    lens = np.ascontiguousarray(lens, np.int32)
    mb, _, _ = layout_dims(lens, page, pool_factor)
    table = np.empty((len(lens), mb), np.int32)
    lib.kvbo_make_paged_layout(_ptr(lens), len(lens), page, pool_factor, seed, _ptr(table))
    return table


def quantize(shape, page, table, lens, max_len, contig, num_blocks):
    table = np.ascontiguousarray(table, np.int32)
    lens = np.ascontiguousarray(lens, np.int32)
    paged = np.zeros((num_blocks, shape.num_kv_heads, page, shape.head_dim), np.int8)
    scales = np.zeros((num_blocks, shape.num_kv_heads), np.float32)
    s = shape_of(shape)
    lib.kvbo_quantize_to_paged_i8(ctypes.byref(s), page, table.shape[1], _ptr(table), _ptr(lens), max_len,
                                  _ptr(np.ascontiguousarray(contig, np.float32)), _ptr(paged), _ptr(scales))
    return paged, scales


def dequantize(shape, page, table, lens, max_len, paged, scales):
    table = np.ascontiguousarray(table, np.int32)
    lens = np.ascontiguousarray(lens, np.int32)
    out = np.zeros((shape.batch, shape.num_kv_heads, max_len, shape.head_dim), np.float32)
    s = shape_of(shape)
    lib.kvbo_dequantize_paged_i8(ctypes.byref(s), page, table.shape[1], _ptr(table), _ptr(lens), max_len,
                                 _ptr(np.ascontiguousarray(paged)), _ptr(np.ascontiguousarray(scales)), _ptr(out))
    return out


def scatter(shape, page, table, lens, max_len, contig, num_blocks):
    table = np.ascontiguousarray(table, np.int32)
    lens = np.ascontiguousarray(lens, np.int32)
    contig = np.ascontiguousarray(contig)
    paged = np.zeros((num_blocks, shape.num_kv_heads, page, shape.head_dim), contig.dtype)
    s = shape_of(shape)
    lib.kvbo_scatter_to_paged(ctypes.byref(s), page, table.shape[1], _ptr(table), _ptr(lens), max_len,
                              contig.dtype.itemsize, _ptr(contig), _ptr(paged))
    return paged


def max_abs_diff(a, b):
    a = np.ascontiguousarray(a, np.float32).ravel()
    b = np.ascontiguousarray(b, np.float32).ravel()
    return lib.kvbo_max_abs_diff(_ptr(a), _ptr(b), a.size)


def auto_part_tokens(batch, num_kv_heads, max_len):
    return lib.kvbo_auto_part_tokens(batch, num_kv_heads, max_len)


def fp16_storage_bound(shape, lens, max_len, q, k32, v32):
    s = shape_of(shape)
    return lib.kvbo_fp16_storage_bound(ctypes.byref(s), _ptr(np.ascontiguousarray(lens, np.int32)), max_len,
                                       _ptr(np.ascontiguousarray(q, np.float32)), _ptr(np.ascontiguousarray(k32)),
                                       _ptr(np.ascontiguousarray(v32)))


def i8_storage_bound(shape, lens, page, table, q, k_scale, v_scale):
    s = shape_of(shape)
    table = np.ascontiguousarray(table, np.int32)
    return lib.kvbo_i8_storage_bound(ctypes.byref(s), _ptr(np.ascontiguousarray(lens, np.int32)), page, table.shape[1],
                                     _ptr(table), _ptr(np.ascontiguousarray(q, np.float32)),
                                     _ptr(np.ascontiguousarray(k_scale)), _ptr(np.ascontiguousarray(v_scale)))


def f32_to_f16_bits(x):
    return lib.kvbo_f32_to_f16(float(x))


def mt64_stream(seed, n):
    state = ctypes.create_string_buffer(312 * 8 + 16)
    lib.kvbo_mt64_seed(state, seed)
    return [lib.kvbo_mt64_next(state) for _ in range(n)]
