"""liblama_hip.so's host logic on the CPU, over a stand-in HIP runtime
(tests/fakehip/fakehip.cpp, loaded through LAMA_HIP_LIB): one "gfx950" device
whose memory is the host heap; launches are counted, not run.  These check
what does not need the kernels' results: every shape plans without an
inconsistent descriptor and issues its counted launches, the plan's kernel
choices and arena sizes, and the error paths -- a failed weight reload keeps
the old weights and plans usable (no launch or copy touches freed device
memory), a failed plan allocation is an error the context recovers from, and
the no-allocation entry point allocates nothing."""
import json
import os
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def fake_lib(tmp_path_factory):
    out = str(tmp_path_factory.mktemp("fakehip") / "libfakehip.so")
    subprocess.run(["g++", "-O1", "-std=c++17", "-shared", "-fPIC", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                    "-o", out, os.path.join(HERE, "fakehip", "fakehip.cpp")], check=True)
    return out


@pytest.fixture(scope="module")
def weights_file(pkg, tmp_path_factory):
    p = str(tmp_path_factory.mktemp("fakew") / "w.safetensors")
    pkg.host_api.synth_weights(p, 0)
    return p


def _scenario(name, fake_lib, weights_file):
    env = dict(os.environ)
    env.pop("FAKEHIP_FAIL_MALLOC_ABOVE", None)
    r = subprocess.run([sys.executable, os.path.join(HERE, "fakehip", "scenarios.py"), name, fake_lib, weights_file],
                       capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0, r.stderr[-3000:]
    return json.loads(r.stdout.strip().splitlines()[-1])


def test_every_shape_plans_and_issues_its_launches(fake_lib, weights_file):
    o = _scenario("plans", fake_lib, weights_file)
    assert o["violations"] == 0
    p = o["plans"]
    for shape, v in p.items():
        # 1 head + 3 downsamplers + 36 FFCs + 3 upsamplers + 1 tail; split
        # transforms add a launch each way
        per_ffc = 10 if v["rfft2"].startswith("lama_rfft2_rows") else 8
        assert v["launch_count"] == 1 + 3 + 36 * per_ffc + 3 + 1, shape
        assert v["issued"] == v["launch_count"], shape
        assert v["conv3x3"] == v["conv3x3g2l"], shape
    # the F(4,3) block shape that covers each bottleneck plane with the fewest blocks
    assert p["512x512"]["conv3x3"] == "lama_conv3x3w4"
    assert p["256x256"]["conv3x3"] == "lama_conv3x3w4n"
    assert p["600x600"]["conv3x3"] == "lama_conv3x3w4q"
    assert p["600x592"]["conv3x3"] == "lama_conv3x3w4q"
    assert p["16x1024"]["conv3x3"] == "lama_conv3x3w4"
    # 1024x1024 and up: Winograd F(2x4, 3x3) (at least two of its blocks per CU),
    # unless its 64-pixel columns overhang the plane by more than an eighth
    # (136 columns in three blocks of 64: F(4,3), in its 8 x 16 blocks there)
    assert p["1024x1024"]["conv3x3"] == "lama_conv3x3w42"
    assert p["1024x1088"]["conv3x3"] == "lama_conv3x3w4q"
    # transforms with the plane shape compiled in, runtime-shaped, split
    assert p["256x256"]["rfft2"] == "lama_rfft2_32" and p["256x256"]["irfft2"] == "lama_irfft2_32"
    assert p["512x512"]["rfft2"] == "lama_rfft2_64"
    assert p["600x600"]["rfft2"] == "lama_rfft2_75" and p["600x600"]["irfft2"] == "lama_irfft2_75"
    assert p["600x592"]["rfft2"] == "lama_rfft2"
    assert p["1024x1024"]["rfft2"] == "lama_rfft2_rows_128"
    # finalize sums 5 partials unsplit, 20 with the 256x256 K split (s = 4)
    assert p["512x512"]["finalize"] == "lama_finalize"
    assert p["256x256"]["finalize"] == "lama_finalize20_g2"  # 128 blocks with one group: two
    # two element groups per thread where one would give 2.5-4 blocks per CU
    assert p["600x600"]["finalize"] == "lama_finalize_g2"
    assert p["1024x1024"]["finalize"] == "lama_finalize"
    # 1x1 activation loads as float4 runs on every bottleneck plane (5625
    # pixels at 600x600 lie 5628 floats apart); K-half tiles where 64 x 64
    # tiles would give at most two workgroups per CU
    assert p["512x512"]["conv1x1"] == "lama_conv1x1_kh"
    assert p["512x512"]["conv1x1res"] == "lama_conv1x1_res_kh"
    assert p["1024x1024"]["conv1x1"] == "lama_conv1x1"
    assert p["1024x1024"]["conv1x1res"] == "lama_conv1x1_res"
    assert p["600x600"]["conv1x1"] == "lama_conv1x1_kh"
    assert p["600x600"]["conv1x1res"] == "lama_conv1x1_res"  # 528 64 x 64 tiles: more than two per CU
    assert p["600x592"]["conv1x1"] == "lama_conv1x1_kh"
    # arena sizes as measured on the MI355X (MiB)
    mib = {k: v["arena"] / 2**20 for k, v in p.items()}
    for shape, want in (("256x256", 69.0), ("512x512", 179.1), ("600x600", 245.8), ("1024x1024", 727.7)):
        assert abs(mib[shape] - want) < 0.1, (shape, mib[shape])
    assert mib["512x512"] < 192  # fits the no-allocation entry point's scratch array
    assert len({v["weights"] for v in p.values()}) == 1
    assert o["inpaint_shape"] == [120, 200, 3]


def test_failed_weight_reload_keeps_the_old_weights_and_plans(fake_lib, weights_file):
    o = _scenario("reload_failure", fake_lib, weights_file)
    assert "hipMalloc(weights)" in o["reload"] and "hipErrorOutOfMemory" in o["reload"], o["reload"]
    assert o["live_kept"]
    assert o["forward_after_failed_reload"] == "ok"
    assert o["forward_after_reload"] == "ok"
    assert o["violations"] == 0


def test_failed_plan_allocation_is_an_error_and_noalloc_allocates_nothing(fake_lib, weights_file):
    o = _scenario("plan_failure", fake_lib, weights_file)
    assert "hipMalloc(activations)" in o["plan"], o["plan"]
    assert o["forward_after_failed_plan"] == "ok"
    assert o["noalloc_512_mallocs"] == 0
    assert o["noalloc_timeline_mallocs"] == 0
    # the scratch array's code object: not loaded at open, loaded once by the first call
    assert o["open_modules"] == 1
    assert o["noalloc_first_modules"] == 1 and o["noalloc_second_modules"] == 0
    assert "captured" in o["noalloc_capture"], o["noalloc_capture"]
    assert "600" in o["noalloc_600"] or "scratch" in o["noalloc_600"], o["noalloc_600"]
    assert o["violations"] == 0
