"""The C ABI without a GPU: libbchip.so loads, exports every function include/bchip.h
declares, and fails cleanly (an error code and a message, no abort) where no gfx950 device
is usable or the GPU is turned off (crates/bc-infer/src/gpu/mod.rs:113-137)."""
import ctypes
import os
import subprocess
import sys

import pytest

import bchip


def test_library_exports_every_declared_function():
    lib = bchip.lib()
    names = bchip.declared_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert lib.bchip_abi_version() == 6


def test_exported_symbols_are_exactly_the_header():
    out = subprocess.run(["nm", "-D", "--defined-only", bchip.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = sorted({l.split()[-1] for l in out.splitlines() if " T bchip_" in l})
    assert exported == bchip.declared_functions()


def test_calls_without_a_context_fail_cleanly():
    lib = bchip.lib()
    rc = lib.bchip_attention(None, None, None, None, 1, None, None, 0, 1, 32, 8, 128, 0, 0.1)
    assert rc == bchip.E_ARG
    assert "context" in bchip.last_error()
    assert lib.bchip_sync(None) == bchip.E_ARG


def _init_in_child(env_extra):
    code = ("import sys, ctypes; sys.path.insert(0, %r); import bchip; h = ctypes.c_void_p(); "
            "rc = bchip.lib().bchip_init(0, ctypes.byref(h)); print(rc, bchip.last_error())") % (
                os.path.dirname(bchip.LIB_PATH))
    env = dict(os.environ, **env_extra)
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=120)
    assert out.returncode == 0, out.stderr
    rc, _, msg = out.stdout.strip().partition(" ")
    return int(rc), msg


def test_gpu_off_switch():
    rc, msg = _init_in_child({"BC_INFER_GPU": "0"})
    assert rc == bchip.E_DISABLED and "BC_INFER_GPU" in msg


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU is present")
def test_no_device_is_an_error_not_a_crash():
    rc, msg = _init_in_child({})
    assert rc in (bchip.E_NODEV, bchip.E_HIP) and msg


def test_cache_capacity_grows_as_the_reference_reserve():
    """Gpu::reserve (gpu/mod.rs:409): at least 256 tokens, doubling, capped by the context
    unless one call needs more."""
    from bchip import grown_capacity
    assert grown_capacity(0, 10, 4096) == 256
    assert grown_capacity(0, 300, 4096) == 300
    assert grown_capacity(256, 257, 4096) == 512
    assert grown_capacity(300, 400, 4096) == 600
    assert grown_capacity(3000, 3001, 4096) == 4096
    assert grown_capacity(4096, 5000, 4096) == 5000
    assert grown_capacity(0, 100, 128) == 128
    for cap, need, context in [(0, 1, 8), (256, 900, 100000), (1 << 20, (1 << 20) + 1, 1 << 22)]:
        got = grown_capacity(cap, need, context)
        assert got >= need and (got >= min(2 * cap, context) or got == need)


def test_stage_rope_frequencies_are_the_reference_f32_values():
    """layers.inv_freq (the host side of a stage) against the oracle's restatement of
    model.rs:208-211 (f32 powf), bit for bit, over the bases and widths the configs use."""
    import numpy as np
    import oracle as O
    from layers import Config, inv_freq
    for base in (10000.0, 500000.0, 1000000.0, 37000.0):
        for rd in (16, 32, 64, 96, 128, 256):
            got = inv_freq(Config(64, 1, 4, 2, rd, rd, base))
            np.testing.assert_array_equal(got.view(np.uint32), O.inv_freq(rd, base).view(np.uint32),
                                          err_msg=f"base {base}, rope_dim {rd}")
