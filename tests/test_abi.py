"""C-ABI and host-logic tests that need no GPU: the library loads, exports every entry point
include/flide_moe.h declares, rejects bad arguments before launching anything, and the Python layer keeps
the reference's signatures and refuses CPU tensors (there is no CPU fallback)."""
from __future__ import annotations

import ctypes
import inspect
import re
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "flide_moe.h"


@pytest.fixture(scope="module")
def lib():
    from flide_amd import _hip

    if not _hip.LIB_PATH.exists():
        from flide_amd import build

        build.build()
    return _hip.load()


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^(?:int|size_t|const char\*)\s+(flide_moe_\w+)\s*\(", text, re.M)))


def test_header_declares_the_path(lib):
    names = _declared()
    for must in ("flide_moe_route", "flide_moe_align", "flide_moe_grouped", "flide_moe_grouped_fp8",
                 "flide_moe_experts", "flide_moe_combine_norm", "flide_moe_combine", "flide_moe_router",
                 "flide_moe_quantize_rows", "flide_moe_rms_norm", "flide_moe_gated_act"):
        assert must in names


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_the_header():
    from flide_amd import _hip

    assert set(_declared()) <= set(_hip.SIGNATURES)


def test_version_and_errors(lib):
    assert lib.flide_moe_version().decode().startswith("flide_moe")
    assert lib.flide_moe_strerror(0) == b"ok"
    assert b"workspace" in lib.flide_moe_strerror(2)
    assert lib.flide_moe_strerror(77) == b"unknown error"


def test_workspace_queries(lib):
    assert lib.flide_moe_align_workspace(0, 128) == 128 * 4
    assert lib.flide_moe_align_workspace(4096, 128) == 128 * 4
    assert lib.flide_moe_align_workspace(4097, 128) == 5 * 128 * 4   # past one workgroup: 1024-pair chunks
    a = lib.flide_moe_experts_workspace(64, 8, 128, 2816, 704, 16, 0)
    b = lib.flide_moe_experts_workspace(8192, 8, 128, 2816, 704, 128, 0)
    c = lib.flide_moe_experts_workspace(8192, 8, 128, 2816, 704, 128, 1)
    assert 0 < a < b < c
    # the workspace holds at least the activation rows [T*k, I] in 16 bits
    assert b >= 8192 * 8 * 704 * 2
    assert lib.flide_moe_experts_workspace(-1, 8, 128, 2816, 704, 16, 0) == 0


def test_bad_arguments_are_rejected_before_any_launch(lib):
    null = None
    # route: k > E, E too large, T < 0
    assert lib.flide_moe_route(null, 128, 4, 8, 9, null, 0, null, null, null) == 1
    assert lib.flide_moe_route(null, 2000, 4, 2000, 8, null, 0, null, null, null) == 1
    assert lib.flide_moe_route(null, 128, -1, 128, 8, null, 0, null, null, null) == 1
    # T == 0 is a no-op success, as in the reference (moe.py:201)
    assert lib.flide_moe_route(null, 128, 0, 128, 8, null, 0, null, null, null) == 0
    # grouped: K not a multiple of 8, unknown dtype, odd N with a gated activation
    args = [null, 64, 1, null, 64 * 64, 64, 64, 60, null, 64, 0, null, null, null, null, 10, 1, 1, 1, 0, 16, 0, null]
    assert lib.flide_moe_grouped(*args) == 1
    args[7] = 64
    args[2] = 9
    assert lib.flide_moe_grouped(*args) == 1
    args[2] = 1
    args[6] = 63
    args[19] = 1
    assert lib.flide_moe_grouped(*args) == 1
    # align: workspace too small
    assert lib.flide_moe_align(null, 100, 16, 16, null, null, null, null, null, 0, null) == 2
    # experts: unknown activation, mismatched fp8 scales
    assert lib.flide_moe_experts(null, 2816, 1, 4, 2816, null, null, 8, null, null, null, null, 128, 704, null, 7, 16,
                                 0, null, 0, null) == 1
    assert lib.flide_moe_experts(null, 2816, 1, 4, 2816, null, null, 8, null, null, ctypes.c_void_p(16), null, 128,
                                 704, null, 1, 16, 0, null, 0, null) == 1
    # combine_norm: H not a multiple of 4
    assert lib.flide_moe_combine_norm(null, 0, null, 10, null, null, 1, null, 10, 1, 3, 10, 2, 1e-6, null) == 1
    # router_norm: H past the LDS staging limit, a misaligned norm weight, an x2 with no norm2 weight
    a16 = ctypes.c_void_p(256)
    rn = [a16, 8200, 4, 8200, 1, a16, a16, 8200, 128, 1e-6, a16, 128, null, 0, null, 0, null]
    assert lib.flide_moe_router_norm(*rn) == 1
    rn[1], rn[3], rn[7] = 2816, 2816, 2816
    rn[5] = ctypes.c_void_p(260)
    assert lib.flide_moe_router_norm(*rn) == 1
    rn[5] = a16
    rn[14] = a16                                                      # x2 without norm2_w
    assert lib.flide_moe_router_norm(*rn) == 1
    # combine_norm_sandwich: k past 8, H past 4096, a missing residual
    sw = [a16, 0, a16, 2816, a16, a16, a16, 2816, a16, null, 0, null, a16, 2816, null, 0, 4, 2816, 9, 1e-6, null]
    assert lib.flide_moe_combine_norm_sandwich(*sw) == 1
    sw[18], sw[17] = 8, 4100
    assert lib.flide_moe_combine_norm_sandwich(*sw) == 1
    sw[17], sw[6] = 2816, null
    assert lib.flide_moe_combine_norm_sandwich(*sw) == 1
    sw[6], sw[16] = a16, 0                                            # T == 0: nothing to do
    assert lib.flide_moe_combine_norm_sandwich(*sw) == 0


def test_signatures_match_the_reference():
    """Parameter names of the public functions, as flide/kernels/moe.py:32-395 and fp8.py:22,46 define them."""
    from flide_amd.kernels import fp8, moe, pointwise

    expect = {
        moe.tile: ["pairs", "fp8", "device"],
        moe.router: ["x", "wr", "wg"],
        moe.route: ["logits", "k", "scale"],
        moe.align: ["ids", "experts", "bm"],
        moe.grouped: ["a", "w", "out", "rows", "blocks", "used", "topk", "by_token", "weights", "tile"],
        moe.grouped_fp8: ["a", "w", "w_scale", "out", "rows", "blocks", "used", "topk", "by_token", "weights", "tile"],
        moe.quantize_experts: ["w"],
        moe.experts: ["x", "w", "top", "ids", "act"],
        moe.moe: ["x", "w", "mm", "swiglu"],
        moe.combine: ["y", "shared", "gate", "k"],
        moe.combine_norm: ["y", "dense", "w1", "w2", "k", "eps"],
        fp8.quantize_rows: ["w"],
        fp8.quantize_tokens: ["x"],
        pointwise.rms_norm: ["x", "w", "eps", "residual", "offset", "dtype"],
        pointwise.geglu: ["a", "b"],
        pointwise.swiglu: ["gu", "n"],
    }
    for fn, names in expect.items():
        params = list(inspect.signature(fn).parameters)
        assert params[:len(names)] == names, (fn.__name__, params)


def test_cpu_tensors_are_refused():
    from flide_amd.kernels import moe

    with pytest.raises(RuntimeError, match="GPU only"):
        moe.route(torch.zeros(4, 8), 2)
    with pytest.raises(RuntimeError, match="GPU only"):
        moe.align(torch.zeros(4, 2, dtype=torch.int32), 8)


def test_tile_choices():
    from flide_amd.kernels import moe

    assert moe.tile(512, False)[0] == 32           # decode: weights streamed through LDS in whole lines
    assert moe.tile(2048, False)[0] == 32
    assert moe.tile(3072, False)[0] == 128         # 16-bit: 128 rows from a few hundred tokens up
    assert moe.tile(65536, False)[0] == 128
    assert moe.tile(512, True)[0] == 32            # float8: 64 rows in between
    assert moe.tile(1024, True)[0] == 64
    assert moe.tile(8192, True)[0] == 64
    assert moe.tile(16384, True)[0] == 128
    assert len(moe.tile(65536, True)) == 5


def test_activation_classification():
    from flide_amd import _hip
    from flide_amd.kernels import moe
    from flide_amd.kernels import pointwise as pw

    def _geglu(a, b):   # the name Gemma's fused decoder calls (flide/backbones/gemma4/fused.py:28)
        return pw.geglu(a, b)

    gemma_act = lambda gu, n: _geglu(gu[:, :n], gu[:, n:])   # noqa: E731  (fused.py:238)
    assert moe._guess_act(gemma_act) == _hip.ACT_GEGLU
    assert moe._guess_act(pw.swiglu) == _hip.ACT_SWIGLU
    assert moe._guess_act(lambda gu, n: torch.relu(gu[:, :n]) * gu[:, n:]) == _hip.ACT_NONE


def test_skewed_workload_calibration():
    """Config 4: the busiest expert takes ~10x the mean load and 10 experts receive nothing."""
    from flide_amd import workloads
    from oracle import moe_oracle as orc

    d = workloads.make_inputs(4, with_weights=False)
    _, ids = orc.route(d["logits"].numpy(), 8)
    counts = np.bincount(ids.reshape(-1), minlength=128)
    mean = counts.sum() / 128
    assert 9.0 <= counts.max() / mean <= 11.0
    assert (counts == 0).sum() == workloads.ZIPF_EMPTY


def test_decode_workload_hits_most_experts():
    from flide_amd import workloads
    from oracle import moe_oracle as orc

    d = workloads.make_inputs(1, with_weights=False)
    _, ids = orc.route(d["logits"].numpy(), 8)
    hit = (np.bincount(ids.reshape(-1), minlength=128) > 0).sum()
    assert 115 <= hit <= 128      # ~126 expected at T = 64, k = 8, E = 128


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus N > 1 (or a multi-rank launch) exits 2 with a message."""
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parent.parent
    r = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
