"""Writes the golden fixtures tests/golden/*.npz from the reference's own CPU code.

Inputs are small seeded numpy arrays; every expected output comes from chipontix/kv-cache-bench's
src/reference.cpp compiled into oracle/_ref/libkvbref.so (make -C oracle ref): attention_reference
for the outputs, make_paged_layout for the block tables (libstdc++'s std::shuffle), and
quantize_to_paged_i8 / dequantize_paged_i8 for the int8 case. The fixtures let the oracle and the
GPU kernels be checked against the reference's own numbers where /root/reference is not mounted.
Run: python tests/golden/make_golden.py
"""
import ctypes
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
import __graft_entry__ as graft  # noqa: E402

oracle = graft.load_oracle()
ref = oracle.ref
assert ref is not None, "oracle/_ref/libkvbref.so is not built (make -C oracle ref)"


class S:
    def __init__(self, b, h, hkv, d):
        self.batch, self.num_heads, self.num_kv_heads, self.head_dim = b, h, hkv, d


def layout(lens, page, seed):
    lens = np.ascontiguousarray(lens, np.int32)
    cap = len(lens) * (max(lens) // page + 2)
    table = np.full(cap, -1, np.int32)
    mb = ctypes.c_int()
    nb = ref.kvbref_make_paged_layout(lens.ctypes.data, len(lens), page, seed, table.ctypes.data, cap, ctypes.byref(mb))
    return table[: len(lens) * mb.value].reshape(len(lens), mb.value), nb


def case(name, shape, lens, page, seed, kind, dist="uniform", q_amp=3.0, dominant=False):
    s = S(*shape)
    g = np.random.Generator(np.random.PCG64(seed))
    L = max(lens)
    kv_shape = (s.batch, s.num_kv_heads, L, s.head_dim)
    if dist == "normal":
        q = (q_amp * g.standard_normal((s.batch, s.num_heads, s.head_dim))).astype(np.float32)
        k, v = g.standard_normal(kv_shape).astype(np.float32), g.standard_normal(kv_shape).astype(np.float32)
    else:
        q = g.uniform(-q_amp, q_amp, (s.batch, s.num_heads, s.head_dim)).astype(np.float32)
        k, v = g.uniform(-1, 1, kv_shape).astype(np.float32), g.uniform(-1, 1, kv_shape).astype(np.float32)
    if kind == "i8":  # magnitudes that differ per 16-token chunk and head, so a misplaced scale shows
        for c in range((L + 15) // 16):
            k[:, :, 16 * c:16 * c + 16] *= np.exp2(-g.uniform(0, 3, (s.batch, s.num_kv_heads, 1, 1))).astype(np.float32)
            v[:, :, 16 * c:16 * c + 16] *= np.exp2(-g.uniform(0, 3, (s.batch, s.num_kv_heads, 1, 1))).astype(np.float32)
    if dominant:
        q[:] = 0
        q[:, :, 0] = 1000.0
        k[:] = 0
        for b, ln in enumerate(lens):
            if ln:
                k[b, :, (7 * b + 3) % ln, 0] = 1.0
    for b, ln in enumerate(lens):  # rows past a length are zero, as the host layer writes them
        k[b, :, ln:] = 0
        v[b, :, ln:] = 0
    table, nb = layout(lens, page, seed)
    lens_a = np.ascontiguousarray(lens, np.int32)
    sc = oracle.scale_of(s.head_dim)
    fix = dict(shape=np.array(shape, np.int32), lens=lens_a, max_len=np.int32(L), page=np.int32(page),
               table=table, num_blocks=np.int32(nb), q=q, kind=np.array(kind))
    if kind == "f16":
        k, v = k.astype(np.float16), v.astype(np.float16)
    if kind == "i8":
        pools = {}
        for nm, src in (("k", k), ("v", v)):
            paged = np.zeros((nb, s.num_kv_heads, page, s.head_dim), np.int8)
            scales = np.zeros((nb, s.num_kv_heads), np.float32)
            ref.kvbref_quantize_to_paged_i8(s.batch, s.num_heads, s.num_kv_heads, s.head_dim, page, table.shape[1], nb,
                                            table.ctypes.data, lens_a.ctypes.data, L, src.ctypes.data, paged.ctypes.data,
                                            scales.ctypes.data)
            deq = np.zeros(kv_shape, np.float32)
            ref.kvbref_dequantize_paged_i8(s.batch, s.num_heads, s.num_kv_heads, s.head_dim, page, table.shape[1], nb,
                                           table.ctypes.data, lens_a.ctypes.data, L, paged.ctypes.data,
                                           scales.ctypes.data, deq.ctypes.data)
            pools[nm] = (paged, scales, deq)
        fix.update(k=k, v=v, k_paged=pools["k"][0], k_scale=pools["k"][1], k_deq=pools["k"][2],
                   v_paged=pools["v"][0], v_scale=pools["v"][1], v_deq=pools["v"][2])
        out = oracle.ref_attention(s, lens_a, L, q, pools["k"][2], pools["v"][2], sc)
    else:
        fix.update(k=k, v=v)
        out = oracle.ref_attention(s, lens_a, L, q, k, v, sc)
    fix["out"] = out
    path = os.path.join(HERE, name + ".npz")
    np.savez_compressed(path, **fix)
    print(f"{path}: out max |x| {np.abs(out).max():.3f}, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    case("gqa4_f32_page16", (3, 8, 2, 128), [37, 1, 20], 16, 101, "f32")
    case("gqa8_f16_d64_empty", (2, 16, 2, 64), [65, 0], 16, 102, "f16")
    case("mha_i8_d64_varied", (2, 4, 4, 64), [33, 16], 16, 103, "i8")
    case("gqa4_f32_normal_page3", (2, 8, 2, 64), [40, 17], 3, 104, "f32", dist="normal", q_amp=1.0)
    case("gqa2_f16_dominant", (2, 8, 4, 64), [29, 50], 16, 105, "f16", dominant=True)
