"""MI355X paged-KV decode attention: the Python face of libkvb_hip.so and libkvb_host.so.

A ctypes mirror of the C ABI in include/kvb_hip.h and include/kvb_host.h, shaped like the
reference's C++ interface (chipontix/kv-cache-bench src/metal_attn.hpp, src/workload.hpp):
``Workload`` builds q and the contiguous K/V cache, ``PagedCache`` its shuffled paged copy (and the
int8 quantisation), ``DeviceCase`` puts both in HBM and runs ``paged_decode`` -> ``paged_reduce``.
Every compute call goes to the HIP library; there is no CPU fallback. If the built libraries are
missing, importing this package raises ImportError.
"""
from __future__ import annotations

import ctypes
import math
import os
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# KVB_BUILD_DIR: libraries built from a mutated copy of the sources (tests/mutation/mutate.py)
BUILD = os.environ.get("KVB_BUILD_DIR") or os.path.join(HERE, "build")

KVB_OK, KVB_EINVAL, KVB_ERUNTIME, KVB_ENODEV = 0, 1, 2, 3
KV_F32, KV_F16, KV_I8 = 0, 1, 2
KV_NAMES = {KV_F32: "f32", KV_F16: "f16", KV_I8: "i8"}
KV_BY_NAME = {v: k for k, v in KV_NAMES.items()}
ELEM_SIZE = {KV_F32: 4, KV_F16: 2, KV_I8: 1}
UNIFORM, NORMAL = 0, 1


def _load(name):
    path = os.path.join(BUILD, name)
    if not os.path.exists(path):
        raise ImportError(f"{path} is not built: run __graft_entry__.build() (make -C kv-cache-bench_amd)")
    return ctypes.CDLL(path)


hip = _load("libkvb_hip.so")
host = _load("libkvb_host.so")

_p = ctypes.c_void_p
_i = ctypes.c_int
_sz = ctypes.c_size_t
_d = ctypes.POINTER(ctypes.c_double)


class PagedArgsC(ctypes.Structure):
    """struct kvb_paged_args (include/kvb_hip.h)."""

    _fields_ = [(n, _i) for n in ("batch", "num_heads", "num_kv_heads", "head_dim", "kv_type", "page_size",
                                  "max_blocks", "max_len", "part_tokens", "share_kv")] + \
               [(n, _p) for n in ("q", "k", "v", "block_table", "seq_lens", "host_seq_lens", "out", "k_scale",
                                  "v_scale", "workspace")] + [("workspace_bytes", _sz)]


class NaiveArgsC(ctypes.Structure):
    """struct kvb_naive_args (include/kvb_hip.h)."""

    _fields_ = [(n, _i) for n in ("batch", "num_heads", "num_kv_heads", "head_dim", "kv_type", "max_len")] + \
               [(n, _p) for n in ("q", "k", "v", "seq_lens", "host_seq_lens", "out")]


class CacheArgsC(ctypes.Structure):
    """struct kvb_cache_args (include/kvb_hip.h)."""

    _fields_ = [(n, _i) for n in ("batch", "num_kv_heads", "head_dim", "kv_type", "page_size", "max_blocks",
                                  "max_len")] + \
               [(n, _p) for n in ("contig", "paged", "scales", "block_table", "seq_lens", "host_seq_lens")]


class DeviceInfoC(ctypes.Structure):
    """struct kvb_device_info_t (include/kvb_hip.h)."""

    _fields_ = [(n, _i) for n in ("runtime_version", "driver_version", "device", "compute_units", "clock_khz",
                                  "memory_clock_khz", "memory_bus_bits", "l2_bytes")] + \
               [("total_memory", _sz), ("free_memory", _sz), ("name", ctypes.c_char * 256),
                ("arch", ctypes.c_char * 64), ("pci_bus_id", ctypes.c_char * 32)]


_PA = ctypes.POINTER(PagedArgsC)
_NA = ctypes.POINTER(NaiveArgsC)
_CA = ctypes.POINTER(CacheArgsC)
_SIGS = {
    "kvb_gpu_available": ([], _i),
    "kvb_device_name": ([ctypes.c_char_p, _sz], _i),
    "kvb_device_info": ([ctypes.POINTER(DeviceInfoC)], _i),
    "kvb_last_error": ([], ctypes.c_char_p),
    "kvb_set_stream": ([_p], _i),
    "kvb_synchronize": ([], _i),
    "kvb_buffer_alloc": ([ctypes.POINTER(_p), _sz], _i),
    "kvb_buffer_free": ([_p], _i),
    "kvb_copy_h2d": ([_p, _p, _sz], _i),
    "kvb_copy_d2h": ([_p, _p, _sz], _i),
    "kvb_fill_bytes": ([_p, _i, _sz], _i),
    "kvb_auto_part_tokens": ([_i, _i, _i], _i),
    "kvb_heads_per_workgroup": ([_i, _i, _i, _i], _i),
    "kvb_paged_max_parts": ([_PA], _i),
    "kvb_paged_workspace_bytes": ([_PA], _sz),
    "kvb_check_paged": ([_PA], _i),
    "kvb_run_paged": ([_PA, _d], _i),
    "kvb_run_paged_steps": ([_PA, _i, _d], _i),
    "kvb_graph_capture_paged": ([_PA, _i, ctypes.POINTER(ctypes.c_void_p)], _i),
    "kvb_graph_launch": ([ctypes.c_void_p, _d], _i),
    "kvb_graph_destroy": ([ctypes.c_void_p], _i),
    "kvb_run_paged_split": ([_PA, _d, _d], _i),
    "kvb_run_paged_loads": ([_PA, _d], _i),
    "kvb_run_empty_grid": ([_i, _i, _d], _i),
    "kvb_paged_kernel_name": ([_PA, _i, ctypes.c_char_p, _sz], _i),
    "kvb_set_pair_mode": ([_i], _i),
    "kvb_set_merge_mode": ([_i], _i),
    "kvb_run_paged_noalloc": ([_PA], _i),
    "kvb_run_naive": ([_NA, _d], _i),
    "kvb_check_naive": ([_NA], _i),
    "kvb_run_attention_fp64": ([_NA, _d], _i),
    "kvb_begin_pipelined": ([], _i),
    "kvb_pipelined_pending": ([], _sz),
    "kvb_end_pipelined": ([_d, _sz, ctypes.POINTER(_sz)], _i),
    "kvb_run_read_bandwidth": ([_p, _sz, _d], _i),
    "kvb_flush_gpu_caches": ([], _i),
    "kvb_write_paged": ([_CA, _d], _i),
    "kvb_check_write_paged": ([_CA], _i),
}
for _name, (_args, _ret) in _SIGS.items():
    _f = getattr(hip, _name)
    _f.argtypes, _f.restype = _args, _ret

_HOST_SIGS = {
    "kvbh_fill_workload": ([_i, _i, _i, _i, _p, _i, _i, ctypes.c_uint64, ctypes.c_float, _i, _i, _p, _p, _p, _p, _p, _i], _i),
    "kvbh_layout_dims": ([_p, _i, _i, ctypes.c_double, _p, _p, _p], _i),
    "kvbh_make_paged_layout": ([_p, _i, _i, ctypes.c_double, ctypes.c_uint64, _p], _i),
    "kvbh_scatter_to_paged": ([_i, _i, _i, _i, _i, _p, _p, _i, _sz, _p, _p], _i),
    "kvbh_quantize_to_paged_i8": ([_i, _i, _i, _i, _i, _p, _p, _i, _p, _p, _p], _i),
    "kvbh_dequantize_paged_i8": ([_i, _i, _i, _i, _i, _p, _p, _i, _p, _p, _p], _i),
    "kvbh_poison_paged": ([_i, _i, _i, _i, _i, _i, _p, _p, _sz, _p, _p], _i),
    "kvbh_mi355x_part_tokens": ([_i, _i, _i, _i, _i, _i, _i, _i], _i),
    "kvbh_mi355x_part_tokens_lens": ([_i, _i, _i, _i, _p, _i, _i, _i], _i),
}
for _name, (_args, _ret) in _HOST_SIGS.items():
    _f = getattr(host, _name)
    _f.argtypes, _f.restype = _args, _ret


class KvbError(RuntimeError):
    """A HIP failure (the reference's std::runtime_error)."""


class KvbInvalidArgument(ValueError):
    """A refusal before any GPU work (the reference's std::invalid_argument)."""


class KvbNoDevice(RuntimeError):
    """No GPU (the reference's metal_available() == false)."""


def check(status, what=""):
    if status == KVB_OK:
        return
    msg = f"{what}: {hip.kvb_last_error().decode()}"
    if status == KVB_EINVAL:
        raise KvbInvalidArgument(msg)
    if status == KVB_ENODEV:
        raise KvbNoDevice(msg)
    raise KvbError(msg)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(_p)


def gpu_available() -> bool:
    return bool(hip.kvb_gpu_available())


def device_name() -> str:
    buf = ctypes.create_string_buffer(256)
    check(hip.kvb_device_name(buf, 256), "device_name")
    return buf.value.decode()


def device_info() -> dict:
    """The device and HIP stack (kvb_device_info): runtime and driver versions, name, architecture,
    PCI bus id, compute units, clocks, memory."""
    d = DeviceInfoC()
    check(hip.kvb_device_info(ctypes.byref(d)), "device_info")
    out = {n: getattr(d, n) for n, _ in DeviceInfoC._fields_}
    for n in ("name", "arch", "pci_bus_id"):
        out[n] = out[n].decode(errors="replace")
    return out


def run_empty_grid(workgroups, threads=256) -> float:
    """GPU ms of one launch of a kernel that does nothing (kvb_run_empty_grid): the dispatch floor."""
    ms = ctypes.c_double()
    check(hip.kvb_run_empty_grid(workgroups, threads, ctypes.byref(ms)), "run_empty_grid")
    return ms.value


def auto_part_tokens(batch, num_kv_heads, max_len) -> int:
    """src/metal_attn.hpp:43-51, through the C ABI."""
    return hip.kvb_auto_part_tokens(batch, num_kv_heads, max_len)


def heads_per_workgroup(shape, kv_type=KV_F16, share_kv=True) -> int:
    """Query heads one paged_decode workgroup serves (kvb_heads_per_workgroup): 32 or 16 where they
    divide the group (f16 and i8 caches), else the largest divisor of the group that is at most 8;
    1 without share_kv."""
    return hip.kvb_heads_per_workgroup(shape.num_heads, shape.num_kv_heads, KV_BY_NAME.get(kv_type, kv_type),
                                       int(share_kv))


def mi355x_part_tokens(shape, max_len, min_groups=256, min_part=256, max_part=4096) -> int:
    """The MI355X partition policy (kvb::mi355x_part_tokens, include/kvb/hip_attn.hpp)."""
    return host.kvbh_mi355x_part_tokens(shape.batch, shape.num_heads, shape.num_kv_heads, shape.head_dim, max_len,
                                        min_groups, min_part, max_part)


def mi355x_part_tokens_for(shape, lens, min_groups=256, min_part=256, max_part=4096) -> int:
    """The MI355X partition policy given the batch's lengths (kvb::mi355x_part_tokens(shape, lens)):
    a ragged batch caps the partition at kvb::ragged_part_cap(max_len): 2048 while the longest sequence
    is under 2 x 3584 tokens, 4096 from 7 x 4096, 3584 between."""
    lens = np.ascontiguousarray(lens, np.int32)
    return host.kvbh_mi355x_part_tokens_lens(shape.batch, shape.num_heads, shape.num_kv_heads, shape.head_dim,
                                             _ptr(lens), min_groups, min_part, max_part)


def mi355x_min_groups(kv_type, head_dim=128) -> int:
    """The policy's workgroup target (kvb::mi355x_min_groups): 256, or 512 when a K or V row is under
    128 bytes (int8 at head_dim 64)."""
    return 512 if ELEM_SIZE[kv_type] * head_dim < 128 else 256


@dataclass
class Shape:
    """src/reference.hpp:17-23."""

    batch: int = 1
    num_heads: int = 32
    num_kv_heads: int = 8
    head_dim: int = 128

    @property
    def group(self):
        return self.num_heads // self.num_kv_heads


class Buffer:
    """Device memory in HBM (kvb_buffer_alloc). Host data moves only through upload()/download()."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        ptr = _p()
        check(hip.kvb_buffer_alloc(ctypes.byref(ptr), self.nbytes), "Buffer")
        self.ptr = ptr.value

    @classmethod
    def from_array(cls, a):
        a = np.ascontiguousarray(a)
        buf = cls(a.nbytes)
        buf.upload(a)
        return buf

    def upload(self, a):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(hip.kvb_copy_h2d(self.ptr, a.ctypes.data_as(_p), a.nbytes), "upload")

    def download(self, dtype, shape):
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes
        check(hip.kvb_copy_d2h(out.ctypes.data_as(_p), self.ptr, out.nbytes), "download")
        return out

    def fill(self, byte):
        check(hip.kvb_fill_bytes(self.ptr, byte, self.nbytes), "fill")

    def free(self):
        if self.ptr:
            hip.kvb_buffer_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Workload:
    """q and the contiguous cache of one decode step (src/workload.hpp:26-88), on the host.

    q ~ q_amp * U(-1,1) and K, V ~ U(-1,1) (``dist="uniform"``, the reference's), or q_amp * N(0,1)
    and N(0,1) (``dist="normal"``, the BASELINE configs); f16 caches hold the values rounded to
    fp16, i8 workloads keep fp32 (PagedCache quantises). Generated by kvbh_fill_workload.
    """

    def __init__(self, shape: Shape, kv_type, lens, seed, q_amp=3.0, keep_f32=False, varied=False,
                 dist="uniform", threads=0):
        self.kv_type = KV_BY_NAME.get(kv_type, kv_type)
        self.lens = np.ascontiguousarray(np.asarray(lens, dtype=np.int32))
        self.shape = Shape(len(self.lens), shape.num_heads, shape.num_kv_heads, shape.head_dim)
        s = self.shape
        self.max_len = int(self.lens.max()) if len(self.lens) else 0
        self.q = np.empty((s.batch, s.num_heads, s.head_dim), np.float32)
        kdt = np.float16 if self.kv_type == KV_F16 else np.float32
        kv_shape = (s.batch, s.num_kv_heads, self.max_len, s.head_dim)
        self.k = np.empty(kv_shape, kdt)
        self.v = np.empty(kv_shape, kdt)
        self.k32 = np.empty(kv_shape, np.float32) if keep_f32 else None
        self.v32 = np.empty(kv_shape, np.float32) if keep_f32 else None
        rc = host.kvbh_fill_workload(s.batch, s.num_heads, s.num_kv_heads, s.head_dim, _ptr(self.lens), self.max_len,
                                     self.kv_type, seed, q_amp, int(varied), NORMAL if dist == "normal" else UNIFORM,
                                     _ptr(self.q), _ptr(self.k), _ptr(self.v), _ptr(self.k32), _ptr(self.v32), threads)
        if rc:
            raise KvbInvalidArgument("Workload: bad shape or lengths")

    @classmethod
    def from_arrays(cls, kv_type, lens, q, k, v):
        """A workload over given arrays: q [B][H][D] f32, k/v [B][Hkv][max_len][D] (f16 or f32)."""
        self = cls.__new__(cls)
        self.kv_type = KV_BY_NAME.get(kv_type, kv_type)
        self.lens = np.ascontiguousarray(np.asarray(lens, dtype=np.int32))
        self.q = np.ascontiguousarray(q, np.float32)
        kdt = np.float16 if self.kv_type == KV_F16 else np.float32
        self.k, self.v = np.ascontiguousarray(k, kdt), np.ascontiguousarray(v, kdt)
        self.shape = Shape(self.q.shape[0], self.q.shape[1], self.k.shape[1], self.q.shape[2])
        self.max_len = self.k.shape[2]
        self.k32 = self.v32 = None
        return self

    def out_floats(self):
        return self.shape.batch * self.shape.num_heads * self.shape.head_dim

    def min_bytes(self):
        """src/workload.hpp:68-74: live K and V plus q and out; int8 scales not included."""
        s = self.shape
        return float(self.lens.sum()) * s.num_kv_heads * s.head_dim * 2 * ELEM_SIZE[self.kv_type] + \
            self.out_floats() * 2 * 4


class PagedCache:
    """The workload's cache in the paged layout (src/workload.hpp:90-146), on the host.

    Shuffled block table over a pool of ceil(live * pool_factor) blocks, or with ``contiguous`` one
    block per sequence in order (page = max_len). int8: quantised per (block, KV head). With
    ``poison``, every pool element no live token owns is NaN (int8: -128, unused scales NaN).
    """

    def __init__(self, w: Workload, page_size, seed=0, contiguous=False, pool_factor=1.0, poison=True,
                 table=None, num_blocks=None):
        s = w.shape
        if table is not None:  # a given block table (e.g. one the reference's make_paged_layout wrote)
            self.table = np.ascontiguousarray(table, np.int32).reshape(s.batch, -1)
            self.page_size, self.max_blocks, self.num_blocks = page_size, self.table.shape[1], int(num_blocks)
        elif contiguous:
            self.page_size, self.max_blocks, self.num_blocks = max(w.max_len, 1), 1, s.batch
            self.table = np.arange(s.batch, dtype=np.int32).reshape(s.batch, 1)
        else:
            mb, live, pool = _i(), _i(), _i()
            if host.kvbh_layout_dims(_ptr(w.lens), s.batch, page_size, pool_factor, ctypes.byref(mb),
                                     ctypes.byref(live), ctypes.byref(pool)):
                raise KvbInvalidArgument("PagedCache: bad layout arguments")
            self.page_size, self.max_blocks, self.num_blocks = page_size, mb.value, pool.value
            self.table = np.empty((s.batch, self.max_blocks), np.int32)
            check_host(host.kvbh_make_paged_layout(_ptr(w.lens), s.batch, page_size, pool_factor, seed,
                                                   _ptr(self.table)), "make_paged_layout")
        pool_shape = (self.num_blocks, s.num_kv_heads, self.page_size, s.head_dim)
        i8 = w.kv_type == KV_I8
        dt = np.int8 if i8 else (np.float16 if w.kv_type == KV_F16 else np.float32)
        self.k = np.zeros(pool_shape, dt)
        self.v = np.zeros(pool_shape, dt)
        self.k_scale = np.zeros((self.num_blocks, s.num_kv_heads), np.float32) if i8 else None
        self.v_scale = np.zeros((self.num_blocks, s.num_kv_heads), np.float32) if i8 else None
        args = (s.batch, s.num_kv_heads, s.head_dim, self.page_size, self.max_blocks)
        if poison:
            for pool, sc in ((self.k, self.k_scale), (self.v, self.v_scale)):
                check_host(host.kvbh_poison_paged(*args, self.num_blocks, _ptr(self.table), _ptr(w.lens),
                                                  ELEM_SIZE[w.kv_type], _ptr(pool), _ptr(sc)), "poison_paged")
        if i8:
            for src, pool, sc in ((w.k, self.k, self.k_scale), (w.v, self.v, self.v_scale)):
                check_host(host.kvbh_quantize_to_paged_i8(*args, _ptr(self.table), _ptr(w.lens), w.max_len, _ptr(src),
                                                          _ptr(pool), _ptr(sc)), "quantize_to_paged_i8")
        else:
            for src, pool in ((w.k, self.k), (w.v, self.v)):
                check_host(host.kvbh_scatter_to_paged(*args, _ptr(self.table), _ptr(w.lens), w.max_len,
                                                      ELEM_SIZE[w.kv_type], _ptr(src), _ptr(pool)), "scatter_to_paged")

    def dequantized(self, w: Workload):
        """int8: the fp32 contiguous values the kernel computes with (dequantize_paged_i8)."""
        s = w.shape
        kd = np.zeros(w.k.shape, np.float32)
        vd = np.zeros(w.v.shape, np.float32)
        for pool, sc, dst in ((self.k, self.k_scale, kd), (self.v, self.v_scale, vd)):
            check_host(host.kvbh_dequantize_paged_i8(s.batch, s.num_kv_heads, s.head_dim, self.page_size,
                                                     self.max_blocks, _ptr(self.table), _ptr(w.lens), w.max_len,
                                                     _ptr(pool), _ptr(sc), _ptr(dst)), "dequantize_paged_i8")
        return kd, vd

    def scale_bytes(self, w: Workload):
        if self.k_scale is None:
            return 0
        blocks = int(((w.lens + self.page_size - 1) // self.page_size).sum())
        return blocks * w.shape.num_kv_heads * 2 * 4


def check_host(rc, what):
    if rc:
        raise KvbInvalidArgument(f"{what} refused its arguments")


class DeviceCase:
    """A workload and its paged cache resident in HBM, ready for paged_decode -> paged_reduce."""

    def __init__(self, w: Workload, c: PagedCache):
        self.w, self.c = w, c
        self.q = Buffer.from_array(w.q)
        self.k = Buffer.from_array(c.k)
        self.v = Buffer.from_array(c.v)
        self.table = Buffer.from_array(c.table if c.table.size else np.zeros(1, np.int32))
        self.lens = Buffer.from_array(w.lens if w.lens.size else np.zeros(1, np.int32))
        self.k_scale = Buffer.from_array(c.k_scale) if c.k_scale is not None else None
        self.v_scale = Buffer.from_array(c.v_scale) if c.v_scale is not None else None
        self.out = Buffer(max(w.out_floats(), 1) * 4)
        self._host_lens = np.ascontiguousarray(w.lens)

    def args(self, part_tokens=0, share_kv=True, workspace: Buffer | None = None, max_len=None) -> PagedArgsC:
        w, c = self.w, self.c
        s = w.shape
        a = PagedArgsC()
        a.batch, a.num_heads, a.num_kv_heads, a.head_dim = s.batch, s.num_heads, s.num_kv_heads, s.head_dim
        a.kv_type, a.page_size, a.max_blocks = w.kv_type, c.page_size, c.max_blocks
        a.max_len = w.max_len if max_len is None else max_len
        a.part_tokens, a.share_kv = part_tokens, int(share_kv)
        a.q, a.k, a.v, a.block_table, a.seq_lens = self.q.ptr, self.k.ptr, self.v.ptr, self.table.ptr, self.lens.ptr
        a.host_seq_lens = self._host_lens.ctypes.data
        a.out = self.out.ptr
        a.k_scale = self.k_scale.ptr if self.k_scale else None
        a.v_scale = self.v_scale.ptr if self.v_scale else None
        if workspace is not None:
            a.workspace, a.workspace_bytes = workspace.ptr, workspace.nbytes
        return a

    def run(self, part_tokens=0, share_kv=True, workspace=None, steps=1) -> float:
        """One (or `steps`) decode step(s); returns GPU ms (0 in pipelined mode)."""
        ms = ctypes.c_double()
        a = self.args(part_tokens, share_kv, workspace)
        check(hip.kvb_run_paged_steps(ctypes.byref(a), steps, ctypes.byref(ms)), "run_paged")
        return ms.value

    def run_split(self, part_tokens=0):
        d, r = ctypes.c_double(), ctypes.c_double()
        a = self.args(part_tokens)
        check(hip.kvb_run_paged_split(ctypes.byref(a), ctypes.byref(d), ctypes.byref(r)), "run_paged_split")
        return d.value, r.value

    def capture_graph(self, part_tokens=0, steps=1) -> "PagedGraph":
        """`steps` decode steps captured into a HIP graph (kvb_graph_capture_paged), with its own
        workspace; launch() replays them. Keep this case alive while the graph is."""
        h = ctypes.c_void_p()
        a = self.args(part_tokens)
        check(hip.kvb_graph_capture_paged(ctypes.byref(a), steps, ctypes.byref(h)), "graph_capture_paged")
        return PagedGraph(h)

    def run_loads(self, part_tokens=0):
        """The decode's loads alone (kvb_run_paged_loads): GPU ms of paged_decode's memory traffic
        with no arithmetic; the output is not written."""
        ms = ctypes.c_double()
        a = self.args(part_tokens)
        check(hip.kvb_run_paged_loads(ctypes.byref(a), ctypes.byref(ms)), "run_paged_loads")
        return ms.value

    def kernel_name(self, part_tokens=0, loads_only=False) -> str:
        """The paged_decode kernel run() (or run_loads()) launches here, as rocprofv3 names it
        (kvb_paged_kernel_name); launches nothing."""
        buf = ctypes.create_string_buffer(512)
        a = self.args(part_tokens)
        check(hip.kvb_paged_kernel_name(ctypes.byref(a), int(loads_only), buf, 512), "paged_kernel_name")
        return buf.value.decode()

    def output(self):
        s = self.w.shape
        return self.out.download(np.float32, (s.batch, s.num_heads, s.head_dim))

    def workspace_bytes(self, part_tokens=0):
        a = self.args(part_tokens)
        return hip.kvb_paged_workspace_bytes(ctypes.byref(a))

    def max_parts(self, part_tokens=0):
        a = self.args(part_tokens)
        return hip.kvb_paged_max_parts(ctypes.byref(a))

    def free(self):
        for b in (self.q, self.k, self.v, self.table, self.lens, self.k_scale, self.v_scale, self.out):
            if b is not None:
                b.free()


class PagedGraph:
    """A captured decode loop (kvb_graph_capture_paged): launch() replays it on the library's stream
    and returns its GPU ms (0 in pipelined mode); free() releases it and its workspace."""

    def __init__(self, handle):
        self.handle = handle

    def launch(self) -> float:
        ms = ctypes.c_double()
        check(hip.kvb_graph_launch(self.handle, ctypes.byref(ms)), "graph_launch")
        return ms.value

    def free(self):
        if self.handle:
            check(hip.kvb_graph_destroy(self.handle), "graph_destroy")
            self.handle = None


def run_attention_fp64(w: Workload, out: Buffer, q: Buffer, k: Buffer, v: Buffer, lens: Buffer) -> float:
    """The reference's fp64 attention_reference on the GPU, over the contiguous f32/f16 cache."""
    return run_naive(w, out, q, k, v, lens, fn="kvb_run_attention_fp64")


def run_naive(w: Workload, out: Buffer, q: Buffer, k: Buffer, v: Buffer, lens: Buffer, fn="kvb_run_naive") -> float:
    """The 3-pass baseline over the contiguous cache (src/metal_attn.mm:211-247)."""
    s = w.shape
    a = NaiveArgsC()
    a.batch, a.num_heads, a.num_kv_heads, a.head_dim = s.batch, s.num_heads, s.num_kv_heads, s.head_dim
    a.kv_type, a.max_len = w.kv_type, w.max_len
    a.q, a.k, a.v, a.seq_lens, a.out = q.ptr, k.ptr, v.ptr, lens.ptr, out.ptr
    host_lens = np.ascontiguousarray(w.lens)
    a.host_seq_lens = host_lens.ctypes.data
    ms = ctypes.c_double()
    check(getattr(hip, fn)(ctypes.byref(a), ctypes.byref(ms)), fn)
    return ms.value


def write_paged(w: Workload, c: PagedCache, contig: Buffer, paged: Buffer, table: Buffer, lens: Buffer,
                scales: Buffer | None = None) -> float:
    """Writes the paged pool (and int8 scales) on the GPU from the contiguous cache in HBM:
    scatter_to_paged for f32/f16 (src/reference.hpp:60-68), quantize_to_paged_i8 for i8 with fp32
    input (src/reference.cpp:32-51). c supplies the layout (page, block table); only live rows are
    written. Returns the kernel's GPU ms."""
    s = w.shape
    a = CacheArgsC()
    a.batch, a.num_kv_heads, a.head_dim, a.kv_type = s.batch, s.num_kv_heads, s.head_dim, w.kv_type
    a.page_size, a.max_blocks, a.max_len = c.page_size, c.max_blocks, w.max_len
    a.contig, a.paged, a.block_table, a.seq_lens = contig.ptr, paged.ptr, table.ptr, lens.ptr
    a.scales = scales.ptr if scales is not None else None
    host_lens = np.ascontiguousarray(w.lens)
    a.host_seq_lens = host_lens.ctypes.data
    ms = ctypes.c_double()
    check(hip.kvb_write_paged(ctypes.byref(a), ctypes.byref(ms)), "write_paged")
    return ms.value


def begin_pipelined():
    check(hip.kvb_begin_pipelined(), "begin_pipelined")


def end_pipelined():
    n = hip.kvb_pipelined_pending()
    ms = (ctypes.c_double * max(n, 1))()
    count = _sz()
    check(hip.kvb_end_pipelined(ms, n, ctypes.byref(count)), "end_pipelined")
    return [ms[i] for i in range(min(count.value, n))]


def flush_gpu_caches():
    check(hip.kvb_flush_gpu_caches(), "flush_gpu_caches")


def synchronize():
    check(hip.kvb_synchronize(), "synchronize")


PAIR_MODES = {"auto": 0, "off": 1, "always": 2}


def set_pair_mode(mode: str) -> str:
    """When a decode workgroup computes two consecutive partitions (kvb_set_pair_mode): "auto",
    "off" or "always" (where allowed). Returns the previous mode."""
    prev = hip.kvb_set_pair_mode(PAIR_MODES[mode])
    if prev < 0:
        raise KvbInvalidArgument(f"set_pair_mode: unknown mode {mode!r}")
    return {v: k for k, v in PAIR_MODES.items()}[prev]


MERGE_MODES = {"auto": 0, "fused": 1, "separate": 2}


def set_merge_mode(mode: str) -> str:
    """Where a decode step merges its partitions (kvb_set_merge_mode): "auto", "fused" (in
    paged_decode, wherever it can) or "separate" (paged_reduce as a second kernel). Returns the
    previous mode."""
    prev = hip.kvb_set_merge_mode(MERGE_MODES[mode])
    if prev < 0:
        raise KvbInvalidArgument(f"set_merge_mode: unknown mode {mode!r}")
    return {v: k for k, v in MERGE_MODES.items()}[prev]


def set_stream(stream):
    """Queues the library's work on `stream` (a hipStream_t as an int or c_void_p; None: the
    library's own), after everything already queued on the previous stream (kvb_set_stream)."""
    check(hip.kvb_set_stream(stream), "set_stream")


def run_read_bandwidth(buf: Buffer) -> float:
    ms = ctypes.c_double()
    check(hip.kvb_run_read_bandwidth(buf.ptr, buf.nbytes // 16 * 16, ctypes.byref(ms)), "run_read_bandwidth")
    return ms.value


def softmax_scale(head_dim):
    return np.float32(1.0) / np.float32(math.sqrt(head_dim))


# The BASELINE configurations (BASELINE.json "configs"): shape, dtype, lengths, page, partition
# (a number where BASELINE names one, "mi355x" = mi355x_part_tokens where it leaves the choice to the
# build, c4's "chosen from length"), pool factor; data N(0,1).
C5_FORCED = (0, 1, 63, 64, 65, 2047, 2048, 2049)


def c5_lengths(seed=5):
    """64 lengths ~ U[1, 16384] from the stated seed, then the forced lengths."""
    g = np.random.Generator(np.random.PCG64(seed))
    return list(g.integers(1, 16385, size=64).astype(int)) + list(C5_FORCED)


CONFIGS = {
    "c1": dict(shape=Shape(1, 32, 8, 128), kv="f32", lens=[512], page=16, part=128, pool=2.0),
    "c2": dict(shape=Shape(8, 32, 8, 128), kv="f16", lens=[4096] * 8, page=16, part=512, pool=1.5),
    "c3": dict(shape=Shape(16, 32, 8, 128), kv="i8", lens=[8192] * 16, page=64, part="mi355x", pool=1.0),
    "c4": dict(shape=Shape(4, 64, 8, 128), kv="f16", lens=[32768] * 4, page=128, part="mi355x", pool=1.25),
    "c5f16": dict(shape=Shape(72, 32, 8, 128), kv="f16", lens=None, page=64, part="mi355x", pool=3.0),
    "c5i8": dict(shape=Shape(72, 32, 8, 128), kv="i8", lens=None, page=64, part="mi355x", pool=3.0),
}


def config_part(cfg, w) -> int:
    """The partition tokens a configuration runs with (its own number, or the MI355X policy for w)."""
    if cfg["part"] == "mi355x":
        return mi355x_part_tokens_for(w.shape, w.lens, min_groups=mi355x_min_groups(w.kv_type, w.shape.head_dim))
    return cfg["part"]


def make_config(name, seed=None, poison=False, threads=0):
    """Workload + PagedCache of a BASELINE configuration (seed defaults to the longest length, the
    reference's Workload seed convention; the table seed is L * 131 + page, bench/bench.cpp:223,244)."""
    cfg = CONFIGS[name]
    lens = cfg["lens"] if cfg["lens"] is not None else c5_lengths()
    L = max(lens)
    seed = L if seed is None else seed
    w = Workload(cfg["shape"], cfg["kv"], lens, seed, q_amp=1.0, dist="normal", threads=threads)
    c = PagedCache(w, cfg["page"], L * 131 + cfg["page"], pool_factor=cfg["pool"], poison=poison)
    return w, c, cfg
