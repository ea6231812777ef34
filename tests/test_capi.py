"""The C ABI on the CPU: both libraries load, export every function that
include/*.h declares, and the HIP library fails loudly -- with a message,
never a CPU fallback -- when no GPU runtime or device is usable."""
import ctypes
import os
import re
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "lama-inpaint-rs_amd", "lib")


def declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lama_\w+)\s*\(", text)))


@pytest.mark.parametrize("header,so", [("lama_host.h", "liblama_host.so"), ("lama_hip.h", "liblama_hip.so")])
def test_every_declared_symbol_is_exported(header, so):
    names = declared(header)
    assert len(names) >= 15
    out = subprocess.run(["nm", "-D", "--defined-only", os.path.join(LIB, so)], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r" T (\w+)$", out, flags=re.M))
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    L = ctypes.CDLL(os.path.join(LIB, so))
    for n in names:
        assert getattr(L, n)


def test_the_hip_library_exports_nothing_but_the_abi():
    out = subprocess.run(["nm", "-D", "--defined-only", os.path.join(LIB, "liblama_hip.so")], capture_output=True,
                         text=True, check=True).stdout
    funcs = set(re.findall(r" T (\w+)$", out, flags=re.M))
    assert funcs == set(declared("lama_hip.h")), funcs ^ set(declared("lama_hip.h"))


def test_the_code_object_is_embedded_for_gfx950():
    blob = open(os.path.join(LIB, "liblama_hip.so"), "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in blob
    for k in [b"lama_conv3x3", b"lama_rfft2", b"lama_irfft2", b"lama_tail", b"lama_convt", b"lama_finalize"]:
        assert k in blob


_PROBE = r"""
import ctypes, os, sys
sys.path.insert(0, {root!r})
import __graft_entry__
pkg = __graft_entry__.load_package()
E = pkg.hip_engine
try:
    E.Engine()
    print("OPENED")
except E.HipError as e:
    print("ERR:" + str(e))
print("VRAM:" + repr(E.vram()))
"""


def _probe(env_extra):
    env = dict(os.environ)
    env.update(env_extra)
    r = subprocess.run([sys.executable, "-c", _PROBE.format(root=ROOT)], capture_output=True, text=True, env=env,
                       timeout=120)
    assert r.returncode == 0, r.stderr
    return r.stdout


def test_open_fails_loudly_with_a_missing_runtime():
    out = _probe({"LAMA_HIP_LIB": "/nonexistent/libamdhip64.so"})
    assert "ERR:" in out and "libamdhip64" in out
    assert "VRAM:None" in out


@pytest.mark.skipif(os.path.exists("/dev/kfd") and os.access("/dev/kfd", os.R_OK | os.W_OK),
                    reason="a GPU is present")
def test_open_fails_loudly_without_a_device():
    out = _probe({})
    assert "ERR:" in out and "OPENED" not in out


def test_missing_library_raises(tmp_path):
    # the ctypes layer refuses to run when liblama_hip.so is absent
    code = (f"import sys; sys.path.insert(0, {ROOT!r}); import __graft_entry__; "
            "pkg = __graft_entry__.load_package(); E = pkg.hip_engine; E.HIP_SO = '/nonexistent.so'\n"
            "try:\n    E.Engine()\nexcept RuntimeError as e:\n    print('RAISED', e)\n")
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert "RAISED" in r.stdout and "not built" in r.stdout


def test_null_context_is_an_error_not_a_crash():
    """Every entry point that takes a context rejects a null one with a
    message (no GPU call is made)."""
    L = ctypes.CDLL(os.path.join(LIB, "liblama_hip.so"))
    err = ctypes.create_string_buffer(256)
    buf = (ctypes.c_float * 16)()
    L.lama_hip_forward.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                   ctypes.c_char_p, ctypes.c_size_t]
    assert L.lama_hip_forward(None, buf, 8, 8, buf, err, 256) == 1
    assert b"null context" in err.value
    L.lama_hip_synchronize.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t]
    err.value = b""
    assert L.lama_hip_synchronize(None, err, 256) == 1 and b"null context" in err.value
    L.lama_hip_launch_count.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
    assert L.lama_hip_launch_count(None, 8, 8) == -1
    L.lama_hip_kernel_name.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_char_p,
                                       ctypes.c_size_t]
    assert L.lama_hip_kernel_name(None, 8, 8, 2, err, 256) == 1
    L.lama_hip_open.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t]
    assert L.lama_hip_open(None, err, 256) == 1 and b"null output" in err.value
    L.lama_hip_close.argtypes = [ctypes.c_void_p]
    L.lama_hip_close(None)


def test_plan_signature_is_the_reference_describe_of_big_lama():
    """lama_hip_plan_signature is model::describe (model.rs:260-274) of the
    plan model::build makes: 29 steps (pad, model.1-4, 18 resblocks, concat,
    3 upsamples, pad, out conv), 4 + 2 * 18 FFC_BN_ACT calls, 18 resblocks."""
    L = ctypes.CDLL(os.path.join(LIB, "liblama_hip.so"))
    L.lama_hip_plan_signature.restype = ctypes.c_char_p
    steps = 1 + 4 + 18 + 1 + 3 + 1 + 1
    assert L.lama_hip_plan_signature().decode() == f"{steps} steps, {4 + 2 * 18} FFC_BN_ACT calls, 18 resblocks"


def test_run_refuses_another_network_before_any_device_work(pkg):
    """hip_engine.run mirrors the Rust binding's plan check: a model whose
    describe() line differs from the backend's plan signature is refused as a
    plan mismatch, before a context is opened (no GPU needed to see it)."""
    E = pkg.hip_engine
    sig = E.plan_signature()
    assert sig.startswith("29 steps, 40 FFC_BN_ACT calls")
    other = "29 steps, 38 FFC_BN_ACT calls, 17 resblocks"
    with pytest.raises(E.HipError, match="plan mismatch"):
        E.run(None, other, np.zeros((4, 8, 8), np.float32), 8, 8)
