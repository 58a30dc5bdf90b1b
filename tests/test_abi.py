"""The C ABI libraries load without a GPU and export every function include/*.h declares."""
import ctypes
import os
import re

import pytest

from conftest import ROOT

BUILD = os.path.join(ROOT, "kv-cache-bench_amd", "build")
HEADERS = {"kvb_hip.h": "libkvb_hip.so", "kvb_host.h": "libkvb_host.so"}


def declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kvbh?_\w+)\s*\(", text)))


@pytest.mark.parametrize("header", sorted(HEADERS))
def test_every_declared_symbol_is_exported(header):
    names = declared(header)
    assert len(names) >= 8, names
    lib = ctypes.CDLL(os.path.join(BUILD, HEADERS[header]))
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"{HEADERS[header]} lacks {missing}"


def test_status_codes_and_no_device_here(kvb):
    assert (kvb.KVB_OK, kvb.KVB_EINVAL, kvb.KVB_ERUNTIME, kvb.KVB_ENODEV) == (0, 1, 2, 3)
    if kvb.gpu_available():
        pytest.skip("a GPU is present")
    ptr = ctypes.c_void_p()
    assert kvb.hip.kvb_buffer_alloc(ctypes.byref(ptr), 64) == kvb.KVB_ENODEV
    assert b"no HIP device" in kvb.hip.kvb_last_error()
