#!/usr/bin/env python3
"""Mutation testing of this build's checks: the reference's scripts/mutation.sh, retargeted.

Each mutant is one textual change to one source file. The harness copies the files a group needs
into a scratch directory, applies the change (it must match exactly once), builds the copy on the
CPU, runs the group's CPU tests against that build, and reports the tests that fail. A mutant is
caught when at least one test fails; the in-tree sources and builds are never touched.

Groups:
  kernel  the reference's kernel mistakes (scripts/mutation.sh:50-59), its kernel-side boundary
          mistakes (:33-36) and mistakes in this build's arithmetic (the fp16 high/low split of q
          and p, the int8 q digits, the V-scale normalisation), planted in the oracle's CPU model
          of this build's split-K kernel (kvbo_split_decode in oracle/kvb_oracle.c, which uses the
          kernel's number formats). They are checked by tests/test_split_model.py, which is the GPU
          parity battery (tests/parity_battery.py) run on that model. No deliberately broken kernel
          runs on a GPU (the GPU boxes forbid it); group hip runs the kernel's own source mutated,
          on the CPU emulation.
  hip     mistakes planted in the shipped kernels' own source (paged_decode_impl.hpp and its
          headers, paged_reduce, the cache writer): the arithmetic of the MFMA kernel (the q and p
          high/low columns, the int8 q digits, the V-scale power of two, the DPP column sums), its
          indexing (the V swizzle, rows inside a page, block ids, the tail mask, the sibling and
          ragged work orders, pair mode) and its merges. The mutated sources are compiled for the
          CPU emulation of gfx950 (tests/kernel_emu) and the GPU test files run on that build
          (tests/kernel_emu/run_gpu_tests.py, stopping at the first failure). Nothing runs on a GPU.
  oracle  mistakes in the checker itself (fp64 attention, layout, quantiser, f16 rounding, RNG,
          storage-error bounds), checked by tests/test_oracle.py: the pins against the reference's
          own build, its golden vectors and closed forms.
  host    the boundary mistakes of the C ABI and the C++ host layer (scripts/mutation.sh:37-41 and
          their neighbours), planted in copies of kv-cache-bench_amd/ and include/, rebuilt with the
          package Makefile (hipcc for runtime.hip), checked by tests/test_host.py, tests/test_abi.py
          and the reference's own C++ test programs compiled against the mutated headers and
          libraries (tests/test_cpp_programs.py, CPU part).

Usage:
  python tests/mutation/mutate.py [GROUP ...] [--only SUBSTR] [--out FILE] [--keep]
  python tests/mutation/mutate.py --check      # every mutation applies exactly once; no build
Exit status 0 when every mutant applied, built and was caught; 1 otherwise.
"""
from __future__ import annotations

import argparse
import os
import re
import shutil
import signal
import subprocess
import sys
import tempfile
import time
from dataclasses import dataclass

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
REFERENCE = "/root/reference"  # the reference's test programs are rebuilt from its sources there
ORACLE_C = "oracle/kvb_oracle.c"
RUNTIME = "kv-cache-bench_amd/csrc/runtime.hip"
KERNEL = "kv-cache-bench_amd/csrc/paged_decode_impl.hpp"
GROUP_TESTS = {
    "kernel": ["tests/test_split_model.py"],
    "hip": ["tests/kernel_emu/run_gpu_tests.py"],
    "oracle": ["tests/test_oracle.py"],
    "host": ["tests/test_host.py", "tests/test_abi.py", "tests/test_cpp_programs.py"],
}
TEST_TIMEOUT = 900  # seconds per mutant's test run


@dataclass(frozen=True)
class Mutant:
    group: str
    name: str
    path: str  # relative to the repository root
    old: str
    new: str


def K(name, old, new):
    return Mutant("kernel", name, ORACLE_C, old, new)


def O(name, old, new):
    return Mutant("oracle", name, ORACLE_C, old, new)


def H(name, path, old, new):
    return Mutant("host", name, path, old, new)


def X(name, old, new, path=KERNEL):
    return Mutant("hip", f"{name} [hip]", path, old, new)


MUTANTS = [
    # ---- the kernel, in the CPU model (reference: scripts/mutation.sh:50-59, 33-36) ----
    K("no online-softmax rescale (corr = 1)",
      "const float corr = exp_ftz(m - m_new);", "const float corr = 1.0f;"),
    K("accumulator rounded to fp16 each step",
      "acc[d] += phi * vrow[i][d];", "acc[d] = round_f16(acc[d] + phi * vrow[i][d]);"),
    K("off-by-one row inside a page",
      "const size_t row = ((blk * Hkv + kvh) * P + t % P) * D;",
      "const size_t row = ((blk * Hkv + kvh) * P + (t + 1) % P) * D;"),
    K("wave merge ignores the max shift in L", "L += wl[w] * wt[w];", "L += wl[w];"),
    K("partition merge drops the last partition",
      "for (int i = 0; i < parts; ++i) {", "for (int i = 0; i < parts - 1; ++i) {"),
    K("block table ignored (logical = physical)",
      "const int32_t id = t / P < j->max_blocks ? bt[t / P] : 0;",
      "const int32_t id = t / P < j->max_blocks ? (int32_t)(t / P) : 0;"),
    K("int8: K scale not applied", "sc[i] *= j->k_scale[blk * Hkv + kvh];", ";"),
    K("int8: K scale of KV head 0 for every head",
      "sc[i] *= j->k_scale[blk * Hkv + kvh];", "sc[i] *= j->k_scale[blk * Hkv];"),
    K("int8: V dequantized with the K scale",
      "vs[i] = j->v_scale[blk * Hkv + kvh];", "vs[i] = j->k_scale[blk * Hkv + kvh];"),
    K("int8: V scale of the sequence's first block for every block",
      "vs[i] = j->v_scale[blk * Hkv + kvh];", "vs[i] = j->v_scale[(size_t)bt[0] * Hkv + kvh];"),
    K("partition merge never writes the output", "out[d] = o * (1.0f / L);", "(void)o;"),
    K("partition merge takes one partition too many at an exact multiple",
      "int parts = (model_len(j, b) + j->part_tokens - 1) / j->part_tokens;",
      "int parts = model_len(j, b) / j->part_tokens + 1;"),
    K("partition merge has no case for an empty sequence", "if (parts == 0) {", "if (0) {"),
    K("query head served by the wrong KV head",
      "const int kvh = h / (s->num_heads / Hkv);", "const int kvh = h % Hkv;"),
    K("softmax scale not applied",
      "const float x = qr[d] * j->scale * (j->kv_type == 0 ? 1.0f : down);",
      "const float x = qr[d] * (j->kv_type == 0 ? 1.0f : down);"),
    # the kernel's number formats (paged_decode_impl.hpp: the q split, the score columns, the fp16
    # split of p and the int8 V-scale normalisation), as the model restates them
    K("fp16 q: low part dropped (q as one fp16 number)",
      "qlo[d] = j->kv_type == 1 ? round_f16(x - qhi[d]) : 0.0f;", "qlo[d] = 0.0f;"),
    K("scores: the power of two that scaled q not undone",
      "sc[i] = (shi + slo) * up;", "sc[i] = shi + slo;"),
    K("int8 q: third digit dropped", "qd2[d] = digit_i8((r1 - qd1[d]) * 128.0f);", "qd2[d] = 0.0f;"),
    K("int8 q: second digit weighted 2^-6 instead of 2^-7",
      "s1 * (1.0f / 128.0f)", "s1 * (1.0f / 64.0f)"),
    K("int8 q: digits of q * scale unscaled (no per-head power of two)",
      "e -= j->kv_type == 2 ? 7 : 14;", "e = j->kv_type == 2 ? 0 : e - 14;"),
    K("p: low fp16 part dropped (p as one fp16 number)",
      "const float plo = j->kv_type == 0 ? 0.0f : round_f16(pv - phi);", "const float plo = 0.0f;"),
    K("int8: p * v_scale split into fp16 without the V-scale normalisation",
      "const float nd = ldexpf(1.0f, -ev);", "const float nd = 1.0f;"),
    K("tail tile drops its last token",
      "const int n = t1 - tt < kModelTile ? t1 - tt : kModelTile;",
      "const int n = t1 - tt < kModelTile ? t1 - tt - 1 : kModelTile;"),
    K("each wave skips every other tile of its stride",
      "tt += j->waves * kModelTile", "tt += 2 * j->waves * kModelTile"),
    K("wave merge weight exp(M - m) instead of exp(m - M)",
      "wt[w] = exp_ftz(wm[w] - M);", "wt[w] = exp_ftz(M - wm[w]);"),
    K("device length not clamped to what the launch holds",
      "return len < 0 ? 0 : len > j->len_cap ? j->len_cap : len;", "return len;"),
    K("partition weight without l (w = exp(m - M))",
      "const float w = ml[2 * i + 1] * exp_ftz(ml[2 * i] - M);", "const float w = exp_ftz(ml[2 * i] - M);"),
    # ---- the shipped kernels' source, run on the CPU emulation (reference: scripts/mutation.sh:50-59) ----
    X("online-softmax rescale dropped (corr = 1)",
      "const float corr = __builtin_amdgcn_exp2f(m - mn);", "const float corr = 1.0f;"),
    X("softmax scale not applied", "qv[j][s] * p.qscale : 0.0f;", "qv[j][s] : 0.0f;"),
    X("q loaded for the wave's first head in every column",
      "hw0 + (qcol ? hh : 0)) * D;", "hw0 + (qcol ? 0 : 0)) * D;"),
    X("head splits: every split serves the workgroup's first heads",
      "const int hw0 = HS == 1 ? h0 : h0 + (wave / TS) * QW;", "const int hw0 = h0;"),
    X("head splits: the wave merge takes the first split's waves for every head",
      "const int w0 = HS == 1 ? 0 : (eh / QW) * TS,", "const int w0 = 0,"),
    # fp16 head splits sharing tiles through LDS (SHL)
    X("shared tiles: both waves of a stream load the K rows",
      "const char* hbase = split ? vbase : kbase;", "const char* hbase = kbase;"),
    X("shared tiles: the second half tile reads the first half's rows",
      "} else {\n                    off += kHalf;\n                }\n                const size_t row0 = ((size_t)max(braw, 0)",
      "} else {\n                    off += 0;\n                }\n                const size_t row0 = ((size_t)max(braw, 0)"),
    X("shared tiles: the V half written without its swizzle",
      "o = SKB + t * D * T::LDS_ESZ + 16 * ((lane % VL) ^ T::vswz(t));", "o = SKB + t * D * T::LDS_ESZ + 16 * (lane % VL);"),
    X("shared tiles: K read back from the slot in another order",
      "rr.k[h][m] = *reinterpret_cast<const uint4*>(slot + ((h * NL + m) * 64 + lane) * 16);",
      "rr.k[h][m] = *reinterpret_cast<const uint4*>(slot + ((m * 2 + h) * 64 + lane) * 16);"),
    X("shared tiles: a wave waits for its own arrival only",
      "want += 128;", "want += 64;"),
    X("fp16 q: low column dropped (q as one fp16 number)",
      "aq16[0][j][s] = hl ? lo : hi;", "aq16[0][j][s] = hl ? (_Float16)0.0f : hi;"),
    X("fp16 q, 16-head waves: low parts dropped",
      "aq16[NA - 1][j][s] = lo;", "aq16[NA - 1][j][s] = (_Float16)0.0f;"),
    X("fp16 q, 16-head waves: one scale for all 16 heads (not one per 8)",
      "for (int x = 1; x < 8; x <<= 1) amax = fmaxf(amax, __shfl_xor(amax, x));",
      "for (int x = 1; x < 16; x <<= 1) amax = fmaxf(amax, __shfl_xor(amax, x));"),
    X("scores: the low column's DPP sum dropped",
      "else s[j] = (S[0][h][i] + dpp<kQuadSwap1>(S[0][h][i])) * f;", "else s[j] = S[0][h][i] * f;"),
    X("scores, 16-head waves: the low part's MFMA dropped",
      "if constexpr (COLH) s[j] = (S[0][h][i] + S[NA - 1][h][i]) * f;", "if constexpr (COLH) s[j] = S[0][h][i] * f;"),
    X("int8 q, 16-head waves: second digit weighted 2^-6 instead of 2^-7",
      "S[NA - 1][h][i] = (float)SB[i] * (1.0f / 128.0f);", "S[NA - 1][h][i] = (float)SB[i] * (1.0f / 64.0f);"),
    X("int8 q, 16-head waves: third digit dropped",
      "S[0][h][i] = __builtin_fmaf((float)SC[i], 1.0f / 16384.0f, (float)SA[i] * 1.0f);",
      "S[0][h][i] = (float)SA[i];"),
    X("int8 q: second digit weighted 2^-6 instead of 2^-7",
      "const float wa = hl ? 1.0f / 128.0f : 1.0f,", "const float wa = hl ? 1.0f / 64.0f : 1.0f,"),
    X("int8 q: third digit dropped", "wb = hl ? 0.0f : 1.0f / 16384.0f;", "wb = 0.0f;"),
    X("int8: K scale not applied", "if constexpr (KIND == KV_I8) f *= FAST ? ksh[h] : r.ks[j];", "(void)ksh;"),
    X("int8: scales of KV head 0 for every head (partition in lanes)",
      "const int soff = lane < nb ? (max(blkv, 0) * Hkv + kvh) * 4 : 0;",
      "const int soff = lane < nb ? (max(blkv, 0) * Hkv) * 4 : 0;"),
    X("p: low fp16 column dropped (p as one fp16 number)",
      "pb16[0][j] = hl ? (_Float16)(pv - (float)hi) : hi;", "pb16[0][j] = hl ? (_Float16)0.0f : hi;"),
    X("p, 16-head waves: low parts dropped",
      "pb16[NA - 1][j] = (_Float16)__builtin_fmaf(pr, xs, -(float)hi);", "pb16[NA - 1][j] = (_Float16)0.0f;"),
    X("P*V, 16-head waves: the low parts' accumulators left out of the wave's state",
      "float4 v = make_float4(a[0] + z[0], a[1] + z[1], a[2] + z[2], a[3] + z[3]);",
      "float4 v = make_float4(a[0], a[1], a[2], a[3]);"),
    X("int8: p * v_scale not normalised by the running power of two",
      "(FAST ? vsh[j >> 2] : r.vs[j]) * vdown : 1.0f;", "(FAST ? vsh[j >> 2] : r.vs[j]) : 1.0f;"),
    X("int8: the V-scale power of two not undone at the end",
      "const float vupf = KIND == KV_I8 ? ldexpf(1.0f, ve) : 1.0f;", "const float vupf = 1.0f;"),
    X("tail mask off by one (the token at the partition end scored)",
      "if (tt + kHalf * (j >> 2) + 4 * q4 + (j & 3) >= t1) s[j] = kNegBig;",
      "if (tt + kHalf * (j >> 2) + 4 * q4 + (j & 3) > t1) s[j] = kNegBig;"),
    X("V tile stored without its swizzle (read with it)", "else sch = ch ^ T::vswz(t);", "else sch = ch;"),
    X("tile-aligned pages: K and V one row later inside the page",
      "const size_t row0 = ((size_t)blk * Hkv + kvh) * P + off;",
      "const size_t row0 = ((size_t)blk * Hkv + kvh) * P + off + 1;"),
    X("tile-aligned pages: the second half tile reads the first half's rows",
      "r.rel[h] = r.rel[0];\n                    off += kHalf;", "r.rel[h] = r.rel[0];\n                    off += 0;"),
    X("the partition's first block for every tile (block ids in lanes)",
      "r.rel[h] = bi - bi0;\n                    braw = lanes ? lane_block(bi - bi0) : bt[bi];",
      "r.rel[h] = bi - bi0;\n                    braw = lanes ? lane_block(0) : bt[bi];"),
    X("any page size: V one row later inside the page",
      "* P + (tvs - vbi * P);", "* P + (tvs + 1 - vbi * P) % P;"),
    X("wave merge weight exp(M - m) instead of exp(m - M)",
      "const float wt = __builtin_amdgcn_exp2f(wml(w).x - M);", "const float wt = __builtin_amdgcn_exp2f(M - wml(w).x);"),
    X("wave merge reads the other waves' rows without their swizzle",
      "wacc(w) + lh * D + 4 * (ed ^ (lh & 7)));", "wacc(w) + lh * D + 4 * ed);"),
    X("partition output not divided by its sum",
      "const float4 r = make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);",
      "const float4 r = make_float4(o.x, o.y, o.z, o.w);"),
    X("fused merge counts only the full partitions",
      "const int nparts = (len + p.part_tokens - 1) / p.part_tokens;", "const int nparts = len / p.part_tokens;"),
    X("fused merge weighs every partition with partition 0's max",
      "add(o, L, partition_weight(ml[j].x, ml[j].y, M), pre[j]);",
      "add(o, L, partition_weight(ml[0].x, ml[j].y, M), pre[j]);"),
    X("fused merge leaves its arrival counter set",
      "        if (threadIdx.x == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);",
      ""),
    X("partition weight without l (w = exp(m - M))",
      "return l * __builtin_amdgcn_exp2f((m - M) * 1.4426950408889634f);",
      "return __builtin_amdgcn_exp2f((m - M) * 1.4426950408889634f);", "kv-cache-bench_amd/csrc/kvb_kernels.hpp"),
    X("pair mode: the second partition starts one tile late",
      "if (cur == 0 && it >= tpp && it < ntiles)", "if (cur == 0 && it > tpp && it < ntiles)"),
    X("sibling workgroups all take the KV head's first head block",
      "bx = (int)((unit % XK) * S + within / 8);", "bx = (int)((unit % XK) * S);"),
    X("ragged order: full partitions numbered from 1",
      "r = WorkItem{64 * e + l, i - __builtin_amdgcn_readlane(excl, l)};",
      "r = WorkItem{64 * e + l, i + 1 - __builtin_amdgcn_readlane(excl, l)};"),
    X("paged_reduce reads partition 0's rows for every partition",
      "ml[j] = p.part_ml[i];\n            v[j] = p.part_out[i * D + d];",
      "ml[j] = p.part_ml[i];\n            v[j] = p.part_out[base * D + d];", "kv-cache-bench_amd/csrc/kernels_misc.hip"),
    X("cache writer: int8 quantiser truncates",
      "__builtin_rintf(x / scale)", "truncf(x / scale)", "kv-cache-bench_amd/csrc/cache_writer.hip"),
    # ---- the checker ----
    O("fp64 reference has no case for an empty sequence (scripts/mutation.sh:36)",
      "len ? (float)(acc[d] / sum) : 0.0f", "(float)(acc[d] / sum)"),
    O("fp64 reference: softmax scale not applied", "p[t] = dot * j->scale;", "p[t] = dot;"),
    O("fp64 reference: max not subtracted before exp",
      "sum += (p[t] = exp(p[t] - mx));", "sum += (p[t] = exp(p[t]));"),
    O("fp64 reference: V read from the K cache",
      "acc[d] += p[t] * load_elem(j->v, base + d, j->f16);", "acc[d] += p[t] * load_elem(j->k, base + d, j->f16);"),
    O("fp64 reference: query head served by the wrong KV head",
      "kvh = h / G, len = j->lens[b];", "kvh = h % s->num_kv_heads, len = j->lens[b];"),
    O("max_abs_diff ignores NaN (scripts/mutation.sh:32)", "if (isnan(e)) return INFINITY;", ""),
    O("auto_part_tokens threshold off by one (scripts/mutation.sh:41)",
      "/ part) < 512) part /= 2;", "/ part) <= 512) part /= 2;"),
    O("f32 -> f16 truncates", "if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) ++h;", ""),
    O("f32 -> f16 ties away from zero", "(rest == 0x1000u && (h & 1u))", "rest == 0x1000u"),
    O("f32 -> f16 subnormals truncate", "if (rest > half || (rest == half && (h & 1u))) ++h;", ""),
    O("f16 -> f32 subnormal exponent off by one",
      "bits = sign | ((uint32_t)(112 - e) << 23) | (man << 13);",
      "bits = sign | ((uint32_t)(113 - e) << 23) | (man << 13);"),
    O("layout: table entries past a sequence's blocks not -1",
      "for (size_t i = 0; i < (size_t)batch * max_blocks; ++i) table[i] = -1;",
      "for (size_t i = 0; i < (size_t)batch * max_blocks; ++i) table[i] = 0;"),
    O("paged_index: off-by-one row inside a page",
      "* page_size + t % page_size) * s->head_dim + d;", "* page_size + (t + 1) % page_size) * s->head_dim + d;"),
    O("scatter reads KV head 0 for every head",
      "src + elem_size * kvbo_contig_index(s, max_len, b, kvh, t, d)",
      "src + elem_size * kvbo_contig_index(s, max_len, b, 0, t, d)"),
    O("quantiser: scale from the signed maximum",
      "const float a = fabsf(contig[kvbo_contig_index(s, max_len, b, kvh, t, d)]);",
      "const float a = contig[kvbo_contig_index(s, max_len, b, kvh, t, d)];"),
    O("quantiser truncates instead of rounding to nearest even",
      "float r = nearbyintf(x / scale);", "float r = truncf(x / scale);"),
    O("quantiser: scale max / 128", "const float scale = amax / 127.0f;", "const float scale = amax / 128.0f;"),
    O("dequantiser: scale of KV head 0 for every head",
      "t / page_size] * s->num_kv_heads + kvh];", "t / page_size] * s->num_kv_heads];"),
    O("mt19937_64: wrong tempering shift", "x ^= x >> 43;", "x ^= x >> 42;"),
    O("partition state drops the last token of a full partition",
      "const int t1 = len < t0 + part_tokens ? len : t0 + part_tokens;",
      "const int t1 = len < t0 + part_tokens ? len : t0 + part_tokens - 1;"),
    O("fp16 storage bound without the V rounding term",
      "return vmax * (u + expm1(2 * E)) + 2e-5;", "return vmax * expm1(2 * E) + 2e-5;"),
    O("fp16 storage bound without the score term",
      "return vmax * (u + expm1(2 * E)) + 2e-5;", "return vmax * u + 2e-5;"),
    O("int8 storage bound without the V rounding term",
      "return vmax * expm1(2 * E) + vq + 2e-5;", "return vmax * expm1(2 * E) + 2e-5;"),
    O("int8 storage bound without the score term",
      "return vmax * expm1(2 * E) + vq + 2e-5;", "return vq + 2e-5;"),
    # ---- the C ABI and the host layer (scripts/mutation.sh:37-41) ----
    H("capacity + 1 accepted", RUNTIME, "(size_t)len > capacity)", "(size_t)len > capacity + 1)"),
    H("exactly the capacity refused", RUNTIME, "(size_t)len > capacity)", "(size_t)len >= capacity)"),
    H("length past max_len accepted", RUNTIME, "len < 0 || len > max_len || (size_t)len", "len < 0 || (size_t)len"),
    H("length check skips the last sequence", RUNTIME,
      "for (int b = 0; b < batch; ++b) {\n        const int len = lens[b];",
      "for (int b = 0; b < batch - 1; ++b) {\n        const int len = lens[b];"),
    H("auto_part_tokens threshold off by one (C ABI)", RUNTIME,
      "/ part) < 512) part /= 2;", "/ part) <= 512) part /= 2;"),
    H("auto_part_tokens threshold off by one (C++ header)", "include/kvb/hip_attn.hpp",
      "/ part) < 512) part /= 2;", "/ part) <= 512) part /= 2;"),
    H("max_abs_diff ignores NaN (C++ header)", "include/kvb/layout.hpp", "if (std::isnan(e)) return INFINITY;", ""),
    H("more than 65535 partitions accepted", RUNTIME, "if (max_parts_of(a) > 65535)", "if (false)"),
    H("int8 cache without scales accepted", RUNTIME,
      "if (a->kv_type == KVB_KV_I8 && (!a->k_scale || !a->v_scale))", "if (false)"),
    H("undersized caller workspace accepted", RUNTIME,
      "if (a->workspace && a->workspace_bytes < workspace_need(a))", "if (false)"),
    H("workspace size without the (m, l) slots", RUNTIME, " + slots * sizeof(float2);", ";"),
    H("head count not a multiple of the KV heads accepted", RUNTIME, "if (H % Hkv != 0)", "if (false)"),
    H("writer: int8 without scales accepted", RUNTIME, "|| (a->kv_type == KVB_KV_I8 && !a->scales)", ""),
    H("host quantiser truncates", "kv-cache-bench_amd/host/layout.cpp",
      "std::nearbyint(x / scale)", "std::trunc(x / scale)"),
    H("host layout: table entries past a sequence's blocks not -1", "kv-cache-bench_amd/host/layout.cpp",
      "L.block_table.assign(seq_lens.size() * size_t(L.max_blocks), -1);",
      "L.block_table.assign(seq_lens.size() * size_t(L.max_blocks), 0);"),
    H("host paged_index: off-by-one row inside a page", "include/kvb/layout.hpp",
      "t % L.page_size) * s.head_dim + d;", "(t + 1) % L.page_size) * s.head_dim + d;"),
]


class NotApplied(Exception):
    pass


def mutated_text(m: Mutant, text: str) -> str:
    n = text.count(m.old)
    if n != 1:
        raise NotApplied(f"{m.path}: the text to replace occurs {n} times")
    return text.replace(m.old, m.new)


def check_all(mutants=MUTANTS) -> list[str]:
    """Problems with the mutant list against the current sources (empty when every mutant applies)."""
    problems, seen = [], set()
    for m in mutants:
        if m.name in seen:
            problems.append(f"duplicate name: {m.name}")
        seen.add(m.name)
        if m.group not in GROUP_TESTS:
            problems.append(f"{m.name}: unknown group {m.group}")
        try:
            with open(os.path.join(ROOT, m.path)) as f:
                mutated_text(m, f.read())
        except (OSError, NotApplied) as e:
            problems.append(f"{m.name}: {e}")
    return problems


def _copy(rel, dst_root, ignore=None):
    src = os.path.join(ROOT, rel)
    dst = os.path.join(dst_root, rel)
    os.makedirs(os.path.dirname(dst), exist_ok=True)
    if os.path.isdir(src):
        shutil.copytree(src, dst, symlinks=True, ignore=ignore)  # copy2: modification times kept
    else:
        shutil.copy2(src, dst)


def prepare(m: Mutant, work: str) -> tuple[dict, str]:
    """Copies what the mutant's group builds, applies the mutant and builds. Returns the
    environment for the test run and the build log."""
    env = dict(os.environ)
    if m.group == "hip":
        skip = shutil.ignore_patterns("__pycache__")
        for d in ("kv-cache-bench_amd/csrc", "kv-cache-bench_amd/host", "include", "tests/kernel_emu"):
            _copy(d, work, skip)  # (with the emulated build's objects: only what the mutant touches rebuilds)
        cmd = ["make", "-C", os.path.join(work, "tests", "kernel_emu"), "-j8", "libs"]
        env["KVB_EMU_BUILD"] = os.path.join(work, "tests", "kernel_emu", "build")
    elif m.group in ("kernel", "oracle"):
        for f in ("oracle/Makefile", "oracle/kvb_oracle.h", ORACLE_C):
            _copy(f, work)
        cmd = ["make", "-C", os.path.join(work, "oracle"), "all"]
        env["KVBO_LIB"] = os.path.join(work, "oracle", "build", "libkvb_oracle.so")
    else:
        skip = shutil.ignore_patterns("__pycache__")
        for d in ("kv-cache-bench_amd", "include"):
            _copy(d, work, skip)
        for f in ("oracle/Makefile", "oracle/kvref.map", "oracle/kvb_oracle.h", "oracle/build/libkvb_oracle.so",
                  "oracle/_ref/libkvref.so"):
            _copy(f, work)
        # the package, then the reference's test programs against the mutated headers and libraries
        pkg = os.path.join(work, "kv-cache-bench_amd")
        cmd = ["bash", "-c", f"make -C {pkg} -j8 && make -C {os.path.join(work, 'oracle')} ref-tests REF={REFERENCE}"]
        env["KVB_BUILD_DIR"] = os.path.join(pkg, "build")
        env["KVB_REF_BIN"] = os.path.join(work, "oracle", "_ref")
    path = os.path.join(work, m.path)
    with open(path) as f:
        text = mutated_text(m, f.read())
    with open(path, "w") as f:
        f.write(text)
    later = time.time() + 2  # newer than every copied object, so make rebuilds what depends on it
    os.utime(path, (later, later))
    b = subprocess.run(cmd, capture_output=True, text=True)
    if b.returncode:
        raise RuntimeError("does not build:\n" + (b.stdout + b.stderr)[-2000:])
    return env, b.stdout


def run_tests(m: Mutant, env: dict, fail_fast=False):
    """(caught, summary). Runs the group's tests in a child process group of its own."""
    if m.group == "hip":  # the GPU test files on the mutated kernels' CPU emulation, to the first failure
        cmd = [sys.executable, os.path.join(ROOT, GROUP_TESTS["hip"][0]), "--build-dir", env["KVB_EMU_BUILD"], "-x",
               "-rf", "-o", "console_output_style=classic"]
    else:
        cmd = [sys.executable, "-m", "pytest", *GROUP_TESTS[m.group], "-q", "-m", "not gpu", "-rf",
               "-p", "no:cacheprovider", "-o", "console_output_style=classic"]
        if fail_fast:
            cmd.append("-x")
    p = subprocess.Popen(cmd, cwd=ROOT, env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                         start_new_session=True)
    try:
        out, _ = p.communicate(timeout=TEST_TIMEOUT)
    except subprocess.TimeoutExpired:
        os.killpg(p.pid, signal.SIGKILL)  # the process group started above, nothing else
        p.communicate()
        return True, f"tests timed out after {TEST_TIMEOUT} s"
    if p.returncode < 0:
        return True, f"test process died with signal {-p.returncode}"
    lines = out.strip().splitlines()
    tail = lines[-1] if lines else ""
    failed = [ln.split(" ", 1)[1].split(" - ", 1)[0] for ln in lines if ln.startswith("FAILED ")]
    failed = [f.replace("tests/", "", 1) for f in failed]
    counts = re.findall(r"(\d+) (passed|failed|error)", tail)
    summary = ", ".join(f"{n} {w}" for n, w in counts) or tail
    # (pytest-xdist stopping at the first failure exits with 2, "interrupted", after its failures)
    if p.returncode == 1 or (p.returncode == 2 and any(w == "failed" and int(n) > 0 for n, w in counts)):
        shown = "; ".join(failed[:3]) + (f"; +{len(failed) - 3} more" if len(failed) > 3 else "")
        return True, f"{summary}: {shown}"
    if p.returncode == 0:
        return False, f"{summary}"
    return False, f"pytest exit {p.returncode}: {tail}"


def run_one(m: Mutant, keep=False, fail_fast=False):
    work = tempfile.mkdtemp(prefix="kvb-mutant-")
    try:
        try:
            env, _ = prepare(m, work)
        except (NotApplied, RuntimeError) as e:
            return "error", str(e)
        caught, summary = run_tests(m, env, fail_fast)
        return ("caught" if caught else "NOT CAUGHT"), summary
    finally:
        if not keep:
            shutil.rmtree(work, ignore_errors=True)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("groups", nargs="*", metavar="GROUP", help=f"any of {', '.join(GROUP_TESTS)} (default: all)")
    ap.add_argument("--only", help="run the mutants whose name contains this text")
    ap.add_argument("--check", action="store_true", help="only check that every mutation applies")
    ap.add_argument("--out", help="also write the report to this file")
    ap.add_argument("--keep", action="store_true", help="keep the scratch directories")
    a = ap.parse_args(argv)
    unknown = [g for g in a.groups if g not in GROUP_TESTS]
    if unknown:
        ap.error(f"unknown group(s) {unknown}; choose from {list(GROUP_TESTS)}")
    problems = check_all()
    if a.check:
        for p in problems:
            print(p)
        print(f"{len(MUTANTS)} mutants, {len(problems)} problems")
        return 1 if problems else 0
    groups = a.groups or list(GROUP_TESTS)
    todo = [m for m in MUTANTS if m.group in groups and (not a.only or a.only in m.name)]
    report, bad = [], 0
    for g in groups:
        ms = [m for m in todo if m.group == g]
        if not ms:
            continue
        head = f"== {g}: {len(ms)} mutants, tests: {' '.join(GROUP_TESTS[g])}"
        print(head, flush=True)
        report.append(head)
        for m in ms:
            t0 = time.time()
            status, summary = run_one(m, a.keep)
            line = f"{m.name}: {status} ({summary}) [{time.time() - t0:.0f} s]"
            print(line, flush=True)
            report.append(line)
            bad += status != "caught"
    tail = f"{len(todo)} mutants, {len(todo) - bad} caught, {bad} not caught or not built"
    print(tail)
    report.append(tail)
    if a.out:
        with open(a.out, "w") as f:
            f.write("\n".join(report) + "\n")
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main())
