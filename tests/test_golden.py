"""Known-answer fixtures (tests/golden/fixtures.npz, written by
tests/golden/make_golden.py from an independent, per-bit restatement of the
reference's fixed-mode stream) against the CPU oracle and the HIP codec.

The GPU tests need neither the oracle nor the generator: the committed
vectors are the expected outputs.
"""

from __future__ import annotations

import os

import numpy as np
import pytest

from conftest import GOLDEN

FIXTURES = os.path.join(GOLDEN, "fixtures.npz")


def load_cases():
    z = np.load(FIXTURES, allow_pickle=False)
    out = []
    for name in z["cases"]:
        name = str(name)
        n, relative, fused, src, epl = (int(v) for v in z[f"{name}.params"])
        out.append(dict(
            name=name, page=z[f"{name}.page"], n=n, relative=relative,
            fused=fused, src=src, epl=epl, eps=float(z[f"{name}.eps"][0]),
            layers=[int(v) for v in z[f"{name}.layers"]] or None,
            eb=np.float32(z[f"{name}.eb"][0]), stream=z[f"{name}.stream"],
            decoded=z[f"{name}.decoded"]))
    return out


CASES = load_cases()
IDS = [c["name"] for c in CASES]


def test_fixture_set_covers_the_hazards():
    names = set(IDS)
    assert {"abs_small", "rel_cross_ref_tile", "rel_specials", "indexed",
            "double_rounding_two", "double_rounding_fused"} <= names
    by = {c["name"]: c for c in CASES}
    # the two quantizer readings must really disagree on this input
    assert not np.array_equal(by["double_rounding_two"]["stream"],
                              by["double_rounding_fused"]["stream"])
    # a stream longer than one reference tile carries header padding
    c = by["rel_cross_ref_tile"]
    nb = (c["n"] + 31) // 32
    assert nb < 2048 and not c["stream"][nb:2048].any()


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_oracle_matches_fixture(oracle, case):
    c = case
    if c["relative"]:
        eb = oracle.relative_bound(c["page"], c["n"], c["eps"], c["layers"],
                                   c["src"], c["epl"])
        assert np.float32(eb) == c["eb"]
    stream = oracle.compress_page(c["page"], c["n"], float(c["eb"]), c["layers"],
                                  c["src"], c["epl"], c["fused"])
    assert np.array_equal(stream, c["stream"])
    dec = oracle.decompress_contiguous(c["stream"], c["n"], float(c["eb"]))
    assert np.array_equal(dec, c["decoded"])


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_hip_codec_matches_fixture(case):
    import ctypes

    import torch

    import kvszp

    c = case
    n = c["n"]
    page = torch.from_numpy(c["page"].view(np.int16).copy()).to("cuda")
    R = 1024 * ((n + 32767) // 32768)
    cap = max(8 * n, R + 128 * ((n + 31) // 32))
    buf = torch.full((cap,), 0xAB, dtype=torch.uint8, device="cuda")
    cfg = kvszp.Config(c["eps"], c["relative"], kvszp.DIM_1D, kvszp.MODE_FIXED,
                       kvszp.TYPE_FLOAT)
    ctx = kvszp.Context(cfg, 0)
    ctx.set_options(c["fused"], kvszp.RATE0_ZERO)
    stream = torch.cuda.current_stream().cuda_stream
    sizes = (ctypes.c_uint64 * 1)()
    bounds = (ctypes.c_float * 1)()
    ins = kvszp.ptr_array([page.data_ptr()])
    outs = kvszp.ptr_array([buf.data_ptr()])
    caps = kvszp.u64_array([cap])
    eps = kvszp.f32_array([c["eps"]])
    if c["layers"]:
        idx = torch.tensor(c["layers"], dtype=torch.long, device="cuda")
        prefix = page.numel() // (c["src"] * c["epl"])
        kvszp.check(ctx.compress_indexed(
            ins, outs, caps, idx.data_ptr(), len(c["layers"]), prefix, c["src"],
            c["epl"], eps, 1, stream, sizes, bounds))
    else:
        kvszp.check(ctx.compress(ins, outs, caps, eps, 1, n, stream, sizes, bounds))
    assert np.float32(bounds[0]) == c["eb"]
    assert sizes[0] == c["stream"].size
    assert np.array_equal(buf[:sizes[0]].cpu().numpy(), c["stream"])

    out = torch.full((n,), 0x7777, dtype=torch.int16, device="cuda")
    kvszp.check(ctx.decompress(
        kvszp.ptr_array([buf.data_ptr()]), kvszp.u64_array([sizes[0]]),
        kvszp.f32_array([bounds[0]]), 1, out.data_ptr(), n, n, stream))
    kvszp.check(ctx.synchronize(stream))
    assert np.array_equal(out.cpu().numpy().view(np.uint16), c["decoded"])
    ctx.close()
