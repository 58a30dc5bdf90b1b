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


def test_package_without_built_libraries_raises(tmp_path):
    """No CPU fallback: with the libraries absent, importing the package fails loudly."""
    import subprocess
    import sys
    code = ("import importlib.util, sys\n"
            f"spec = importlib.util.spec_from_file_location('kvb', {os.path.join(ROOT, 'kv-cache-bench_amd', '__init__.py')!r})\n"
            "m = importlib.util.module_from_spec(spec)\n"
            "try:\n"
            "    spec.loader.exec_module(m)\n"
            "except ImportError as e:\n"
            "    print('ImportError:', e); sys.exit(3)\n"
            "sys.exit(0)\n")
    env = dict(os.environ, KVB_BUILD_DIR=str(tmp_path))
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=120)
    assert r.returncode == 3, r.stdout + r.stderr
    assert "libkvb_hip.so is not built" in r.stdout
