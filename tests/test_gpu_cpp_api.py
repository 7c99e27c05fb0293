"""The C++ header driven by a compiled C++ caller (tests/cpp/cpp_api_caller.cpp,
built next to the library by __graft_entry__.build()), the way the
reference's own C++ harnesses drive its header: caller-owned buffers,
fp8mega::layout, fill_weights_lane, launch_full, read_status.  Its fp32
output must equal the Python operator API's (over the C ABI) bit for bit on
the same inputs, and the Python path is itself checked against the oracle."""
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

import mini_mega_amd as mm

import moe_case as mc

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "_build",
                   "cpp_api_caller")


def _say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    torch.cuda.set_device(0)
    mm.lib()
    yield


@pytest.mark.parametrize("E,K,H,I,T", [(16, 4, 512, 256, 96), (64, 8, 1024, 512, 300)])
def test_cpp_caller_matches_python_api(tmp_path, E, K, H, I, T):
    assert os.path.exists(BIN), f"{BIN} is missing: run __graft_entry__.build() first"
    s1, s2 = 17, 91
    _say(f"C++ caller E={E} K={K} H={H} I={I} T={T}")
    rng = np.random.default_rng(T)
    x = (torch.randn((T, H), generator=torch.Generator().manual_seed(T)) * 0.5).to(
        torch.float8_e4m3fn).view(torch.uint8).numpy()
    idx = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int64)
    wts = rng.random((T, K)).astype(np.float32)
    wts /= wts.sum(axis=1, keepdims=True)
    (tmp_path / "dims.txt").write_text(f"{E} {K} {H} {I} {T} {s1} {s2}\n")
    x.tofile(tmp_path / "x.bin")
    idx.tofile(tmp_path / "idx.bin")
    wts.tofile(tmp_path / "wts.bin")
    p = subprocess.run([BIN, str(tmp_path)], capture_output=True, text=True, timeout=120)
    _say(f"  C++ caller: rc={p.returncode} {p.stdout.strip()} {p.stderr.strip()}")
    assert p.returncode == 0, p.stderr
    y_cpp = np.fromfile(tmp_path / "y.bin", dtype=np.float32).reshape(T, H)

    # the same layer through the Python operator API and the C ABI
    L = mm.lib()
    stream = torch.cuda.current_stream().cuda_stream
    w1 = torch.empty((E, 2 * I, H), dtype=torch.uint8, device="cuda")
    w2 = torch.empty((E, H, I), dtype=torch.uint8, device="cuda")
    assert L.mm_fill_weights_lane(w1.data_ptr(), E * 2 * I, H, s1, stream) == 0
    assert L.mm_fill_weights_lane(w2.data_ptr(), E * H, I, s2, stream) == 0
    c = mc.Case(E, K, H, I, T, x, None, idx, wts, w1.view(torch.float8_e4m3fn), None,
                w2.view(torch.float8_e4m3fn), None)
    r = mc.run_layer(c)
    mc.check_routing(c, r)
    mc.check_reduce(c, r)
    mc.check_e2e(c, r)
    assert np.array_equal(y_cpp.view(np.uint32), r.y32.view(np.uint32)), \
        "C++ caller output differs from the Python API's"
    assert p.stdout.split()[0] == "ok" and f"slots={T * K}" in p.stdout
