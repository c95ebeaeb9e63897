"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle still reproduces every fixture exactly (a regression guard on the checker itself).
GPU: the HIP path matches the fixtures -- routing ids, align's rows/blocks/used/counts and the FP8
quantisation bytes bit-exactly; expert rows within 1e-2 (bf16) / 3e-2 (fp8) relative."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import moe_oracle as orc
from tests.helpers import assert_close

GOLD = Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLD / f"{name}.npz", allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


# ------------------------------------------------------------------------------------------- CPU side
def test_oracle_reproduces_route_fixture():
    d = load("route")
    w, ids = orc.route(d["logits"], int(d["k"]), d["scale"])
    np.testing.assert_array_equal(ids, d["ids"])
    np.testing.assert_array_equal(w, d["w"])


def test_oracle_reproduces_align_fixture():
    d = load("align")
    for bm in (16, 64):
        al = orc.align(d["ids"], int(d["E"]), bm)
        np.testing.assert_array_equal(al["rows"], d[f"rows_bm{bm}"])
        np.testing.assert_array_equal(al["blocks"], d[f"blocks_bm{bm}"])
        np.testing.assert_array_equal(al["used"], d[f"used_bm{bm}"])
    assert (d["counts"][7] == 0) and d["counts"][3] > 150      # the fixture's empty and hot experts


def test_oracle_reproduces_experts_fixtures():
    d = load("experts_bf16")
    y = orc.experts(d["x"], d["w_gu"], d["w_d"], d["top"], d["ids"], int(d["inter"]), "geglu", "bf16")
    np.testing.assert_array_equal(y, d["y"])
    f = load("experts_fp8")
    y8 = orc.experts_fp8(f["x"], orc.e4m3fn_decode(f["q_gu"]), f["s_gu"], orc.e4m3fn_decode(f["q_d"]), f["s_d"],
                         f["top"], f["ids"], int(f["inter"]))
    np.testing.assert_array_equal(y8, f["y"])


# ------------------------------------------------------------------------------------------- GPU side
def _bf16(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16).cuda()


@pytest.mark.gpu
def test_gpu_route_fixture():
    from flide_amd.kernels import moe

    d = load("route")
    w, ids = moe.route(torch.from_numpy(d["logits"]).cuda(), int(d["k"]), torch.from_numpy(d["scale"]).cuda())
    np.testing.assert_array_equal(ids.cpu().numpy(), d["ids"])
    np.testing.assert_allclose(w.cpu().numpy(), d["w"], rtol=1e-5, atol=1e-7)


@pytest.mark.gpu
def test_gpu_align_fixture():
    from flide_amd.kernels import moe

    d = load("align")
    E = int(d["E"])
    for bm in (16, 64):
        counts = torch.empty(E, dtype=torch.int32, device="cuda")
        rows, blocks, used = moe.align(torch.from_numpy(d["ids"]).cuda(), E, bm, counts=counts)
        u = int(used.item())
        assert u == int(d[f"used_bm{bm}"][0])
        np.testing.assert_array_equal(rows.cpu().numpy()[:u], d[f"rows_bm{bm}"][:u])
        np.testing.assert_array_equal(blocks.cpu().numpy()[:u // bm], d[f"blocks_bm{bm}"][:u // bm])
        np.testing.assert_array_equal(counts.cpu().numpy(), d["counts"])


@pytest.mark.gpu
def test_gpu_experts_bf16_fixture():
    from flide_amd.kernels import moe
    from flide_amd.kernels import pointwise as pw

    d = load("experts_bf16")
    k = int(d["k"])
    w = {"experts": _bf16(d["w_gu"]), "experts_down": _bf16(d["w_d"]), "inter": int(d["inter"])}
    top, ids = moe.route(torch.from_numpy(d["logits"]).cuda(), k)
    np.testing.assert_array_equal(ids.cpu().numpy(), d["ids"])
    y = moe.experts(_bf16(d["x"]), w, top, ids, lambda gu, n: pw.geglu(gu[:, :n], gu[:, n:]))
    assert_close(y.float().cpu().numpy(), d["y"], 1e-2, "golden experts bf16")
    out = moe.combine_norm(y, _bf16(d["dense"]), _bf16(d["w1"]), _bf16(d["w2"]), k, 1e-6)
    assert_close(out.float().cpu().numpy(), d["out"], 1e-2, "golden combine_norm")


@pytest.mark.gpu
def test_gpu_experts_fp8_fixture():
    from flide_amd.kernels import fp8, moe
    from flide_amd.kernels import pointwise as pw

    f = load("experts_fp8")
    k = int(f["k"])
    q = lambda a: torch.from_numpy(np.ascontiguousarray(a)).view(torch.float8_e4m3fn).cuda()  # noqa: E731
    w = {"experts": q(f["q_gu"]), "experts_down": q(f["q_d"]), "inter": int(f["inter"]),
         "experts_scale": torch.from_numpy(f["s_gu"]).cuda(), "experts_down_scale": torch.from_numpy(f["s_d"]).cuda()}
    x = _bf16(f["x"])
    qx, sx = fp8.quantize_tokens(x)
    np.testing.assert_array_equal(qx.cpu().view(torch.uint8).numpy(), f["qx"])
    np.testing.assert_array_equal(sx.cpu().numpy(), f["sx"])
    top, ids = moe.route(torch.from_numpy(f["logits"]).cuda(), k)
    y = moe.experts(x, w, top, ids, lambda gu, n: pw.geglu(gu[:, :n], gu[:, n:]))
    assert_close(y.float().cpu().numpy(), f["y"], 3e-2, "golden experts fp8")
