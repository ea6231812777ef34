"""Scenarios for tests/test_fake_hip.py, one per process (the engine loads its
HIP runtime once per process): `python scenarios.py <name> <fake lib>
<weights file>` runs liblama_hip.so over the stand-in runtime of fakehip.cpp
and prints one JSON object with what it observed."""
import ctypes
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

name, fake_path, weights = sys.argv[1], sys.argv[2], sys.argv[3]
os.environ["LAMA_HIP_LIB"] = fake_path
import __graft_entry__  # noqa: E402

pkg = __graft_entry__.load_package()
E, H = pkg.hip_engine, pkg.host_api
fake = ctypes.CDLL(fake_path)
fake.fakehip_launches.argtypes = [ctypes.c_char_p]
fake.fakehip_launches.restype = ctypes.c_long
fake.fakehip_live_bytes.restype = ctypes.c_long
fake.fakehip_modules.restype = ctypes.c_long
out = {}


def run_plans():
    eng = E.Engine()
    eng.load_weights(H.Store(weights))
    shapes = [(64, 64), (128, 96), (256, 256), (512, 512), (600, 600), (600, 592), (1024, 1024), (16, 1024),
              (8, 8), (64, 1024), (1024, 1088)]
    res = {}
    for h, w in shapes:
        before = fake.fakehip_launches(None)
        eng.forward(np.zeros((4, h, w), np.float32))
        issued = fake.fakehip_launches(None) - before
        arena, wbytes = eng.plan_bytes(h, w)
        res[f"{h}x{w}"] = {
            "launch_count": eng.launch_count(h, w), "issued": issued, "arena": arena, "weights": wbytes,
            "conv3x3": eng.kernel_name(h, w, "conv3x3"), "conv3x3g2l": eng.kernel_name(h, w, "conv3x3g2l"),
            "rfft2": eng.kernel_name(h, w, "rfft2"), "irfft2": eng.kernel_name(h, w, "irfft2"),
            "conv1x1": eng.kernel_name(h, w, "conv1x1"), "finalize": eng.kernel_name(h, w, "finalize"),
            "conv1x1res": eng.kernel_name(h, w, "conv1x1res"),
        }
    out["plans"] = res
    # the u8 flow and the isolated SpectralTransform plan at two shapes
    rgb = np.zeros((120, 200, 3), np.uint8)
    mask = np.zeros((120, 200), np.uint8)
    u8 = eng.inpaint(rgb, mask)
    out["inpaint_shape"] = list(u8.shape)
    eng.spectral(0, np.zeros((384, 64, 64), np.float32))
    eng.spectral(17, np.zeros((384, 75, 75), np.float32))
    eng.close()


def run_reload_failure():
    eng = E.Engine()
    store = H.Store(weights)
    eng.load_weights(store)
    eng.forward(np.zeros((4, 64, 64), np.float32))
    live = fake.fakehip_live_bytes()
    os.environ["FAKEHIP_FAIL_MALLOC_ABOVE"] = str(100 << 20)
    try:
        eng.load_weights(store)
        out["reload"] = "succeeded"
    except E.HipError as e:
        out["reload"] = str(e)
    del os.environ["FAKEHIP_FAIL_MALLOC_ABOVE"]
    out["live_kept"] = fake.fakehip_live_bytes() == live
    # the old weights and the cached 64x64 plan still serve
    eng.forward(np.zeros((4, 64, 64), np.float32))
    out["forward_after_failed_reload"] = "ok"
    eng.load_weights(store)  # a successful reload replaces both
    eng.forward(np.zeros((4, 64, 64), np.float32))
    out["forward_after_reload"] = "ok"
    eng.close()


def run_plan_failure():
    # opening a context loads the kernels' code object only; the no-allocation
    # entry point's array (its own code object) waits for that entry's first call
    modules = fake.fakehip_modules()
    eng = E.Engine()
    out["open_modules"] = fake.fakehip_modules() - modules
    eng.load_weights(H.Store(weights))
    os.environ["FAKEHIP_FAIL_MALLOC_ABOVE"] = str(50 << 20)
    try:
        eng.forward(np.zeros((4, 512, 512), np.float32))
        out["plan"] = "succeeded"
    except E.HipError as e:
        out["plan"] = str(e)
    del os.environ["FAKEHIP_FAIL_MALLOC_ABOVE"]
    eng.forward(np.zeros((4, 512, 512), np.float32))
    out["forward_after_failed_plan"] = "ok"
    # the no-allocation entry point: 512x512 runs in the scratch array, 600x600 is refused
    d_in, d_out = eng.malloc(4 * 600 * 600 * 4), eng.malloc(3 * 600 * 600 * 4)
    mallocs, modules = fake.fakehip_mallocs(), fake.fakehip_modules()
    eng.forward_device_noalloc(d_in, 512, 512, d_out)
    out["noalloc_512_mallocs"] = fake.fakehip_mallocs() - mallocs
    out["noalloc_first_modules"] = fake.fakehip_modules() - modules
    modules = fake.fakehip_modules()
    eng.forward_device_noalloc(d_in, 512, 512, d_out)
    out["noalloc_second_modules"] = fake.fakehip_modules() - modules
    # with the launch timeline on, still no allocation
    eng.timeline(True)
    mallocs = fake.fakehip_mallocs()
    eng.forward_device_noalloc(d_in, 512, 512, d_out)
    out["noalloc_timeline_mallocs"] = fake.fakehip_mallocs() - mallocs
    eng.timeline(False)
    # a stream under capture is refused
    os.environ["FAKEHIP_CAPTURING"] = "1"
    try:
        eng.forward_device_noalloc(d_in, 512, 512, d_out)
        out["noalloc_capture"] = "succeeded"
    except E.HipError as e:
        out["noalloc_capture"] = str(e)
    del os.environ["FAKEHIP_CAPTURING"]
    try:
        eng.forward_device_noalloc(d_in, 600, 600, d_out)
        out["noalloc_600"] = "succeeded"
    except E.HipError as e:
        out["noalloc_600"] = str(e)
    eng.free(d_in)
    eng.free(d_out)
    eng.close()


{"plans": run_plans, "reload_failure": run_reload_failure, "plan_failure": run_plan_failure}[name]()
out["violations"] = fake.fakehip_violations()
print(json.dumps(out))
