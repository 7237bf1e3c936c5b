"""Pins the scalar C oracle of the 4-bit codec (usaf/quantization.py:21-132).

Checks: hand-derived known-answer vectors (tests/golden/q4_kat.json), numpy's
IEEE float16 conversions and arithmetic (a library independent of the
oracle), a second restatement in torch CPU ops (oracle/codec_torch.py),
and invariants the format fixes (code range, argmin/argmax codes, the
reconstruction bound).
"""
import json
import os

import numpy as np
import pytest
import torch

import oracle
from oracle.codec_torch import dequant_opseq, quantize_opseq

KAT = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "q4_kat.json")))


def _kat(name):
    return next(k for k in KAT if k["name"] == name)


def test_half_to_float_exhaustive():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.half_to_float(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_float_to_half_matches_numpy_rne():
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 5, 20000),
        # exact ties between neighbouring halves (normal and subnormal ranges)
        (np.arange(1, 2048, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -24),
        (np.arange(1024, 2048, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -10),
        np.array([65504, 65519.99, 65520, 1e-12, 2.0 ** -25, 2.0 ** -25 * 1.0000001, 0.0, -0.0],
                 dtype=np.float32),
    ])
    ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([oracle.float_to_half(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, ref)


def test_dequant_arithmetic_exhaustive_over_scales():
    # Every finite fp16 scale x every code, random zeros: the oracle's
    # fp16(fp16(q*s)+z) equals numpy float16 arithmetic (mul then add, each rounded).
    s_all = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    s_all = s_all[np.isfinite(s_all.view(np.float16))]
    rng = np.random.default_rng(1)
    G = s_all.size
    gs = 32
    codes = rng.integers(0, 16, size=(G, gs), dtype=np.uint8)
    codes[:, :16] = np.arange(16, dtype=np.uint8)  # every code for every scale
    z = rng.standard_normal(G).astype(np.float16)
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).view(np.int8)
    got = oracle.dequant(packed, s_all, z.view(np.uint16), G * gs, gs)
    with np.errstate(over="ignore", invalid="ignore"):
        ref = (codes.astype(np.float16) * s_all.view(np.float16)[:, None]) + z[:, None]
    ref = ref.reshape(-1)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got.view(np.float16)), nan)
    assert np.array_equal(got[~nan], ref.view(np.uint16)[~nan])


def test_double_rounding_kat():
    # A fused multiply-add (one rounding) is a plausible mistake; these cases separate the two.
    for q, s, z, two, one in _kat("double_rounding")["cases"]:
        got = oracle.dequant(np.array([[q]], dtype=np.int8), np.array([s], np.uint16), np.array([z], np.uint16), 1, 1)
        assert int(got[0]) == two and two != one


@pytest.mark.parametrize("name", ["ramp", "pad_tail", "constant", "tiny", "odd_gs3"])
def test_quantize_kat(name):
    k = _kat(name)
    p, s, z = oracle.quantize(np.array(k["x"], dtype=np.float32), k["group_size"])
    assert p.tolist() == k["packed"]
    assert s.tolist() == k["scale"]
    assert z.tolist() == k["zero"]


@pytest.mark.parametrize("name", ["ramp", "constant", "odd_gs3_dequant_layout"])
def test_dequant_kat(name):
    k = _kat(name)
    p = np.array(k["packed"], dtype=np.int8)
    got = oracle.dequant(p, np.array(k["scale"], np.uint16), np.array(k["zero"], np.uint16),
                         len(k["dequant_f16"]), k["group_size"])
    assert got.tolist() == k["dequant_f16"]


@pytest.mark.parametrize("shape,gs", [((768, 2048), 128), ((3, 333), 128), ((7,), 128), ((5, 7), 3),
                                      ((1000,), 64), ((129,), 128), ((2, 255), 5)])
def test_oracle_matches_torch_restatement(shape, gs):
    g = torch.Generator().manual_seed(1234)
    w = (torch.randn(shape, generator=g) * 0.02).half()
    p_t, s_t, z_t = quantize_opseq(w, gs)
    p_o, s_o, z_o = oracle.quantize(w.float().numpy(), gs)
    assert np.array_equal(p_o, p_t.numpy())
    assert np.array_equal(s_o, s_t.numpy().view(np.uint16))
    assert np.array_equal(z_o, z_t.numpy().view(np.uint16))
    d_t = dequant_opseq(p_t, s_t, z_t, w.shape, gs)
    d_o = oracle.dequant(p_o, s_o, z_o, w.numel(), gs)
    assert np.array_equal(d_o, d_t.numpy().reshape(-1).view(np.uint16))


def test_quantize_invariants_cfg0():
    # cfg0: W [768, 2048] ~ N(0, 0.02), fp16
    g = torch.Generator().manual_seed(1234)
    w = (torch.randn(768, 2048, generator=g) * 0.02).half().float().numpy().reshape(-1)
    p, s, z = oracle.quantize(w, 128)
    assert p.shape == (12288, 64) and s.shape == (12288,)
    codes = np.empty((12288, 128), dtype=np.uint8)
    pu = p.view(np.uint8)
    codes[:, 0::2] = pu & 0xF
    codes[:, 1::2] = pu >> 4
    x = w.reshape(12288, 128)
    assert codes.max() <= 15
    rows = np.arange(12288)
    assert np.all(codes[rows, x.argmin(1)] == 0)
    assert np.all(codes[rows, x.argmax(1)] == 15)
    # reconstruction: |x - xhat| <= scale/2 (quantization) + fp16 rounding of scale/zero/output
    xh = oracle.dequant(p, s, z, w.size, 128).view(np.float16).astype(np.float32).reshape(12288, 128)
    sc32 = (x.max(1) - x.min(1)) / 15
    bound = sc32 / 2 + 15 * np.abs(sc32 - s.view(np.float16).astype(np.float32)) \
        + np.abs(x.min(1) - z.view(np.float16).astype(np.float32)) + 2 * 2.0 ** -11 * np.abs(x).max(1) + 1e-7
    assert np.all(np.abs(x - xh).max(1) <= bound)


def test_dequant_bf16_is_torch_conversion():
    g = torch.Generator().manual_seed(5)
    w = torch.randn(4096, generator=g).half()
    p, s, z = oracle.quantize(w.float().numpy(), 128)
    f16 = oracle.dequant(p, s, z, w.numel(), 128)
    bf = oracle.dequant(p, s, z, w.numel(), 128, out_dtype="bf16")
    ref = torch.from_numpy(f16.view(np.float16)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bf, ref)
    for h in [0x7C00, 0xFC00, 0x7E00, 0x0001, 0x03FF, 0x8001]:
        ref_h = torch.tensor([h], dtype=torch.int32).to(torch.int16).view(torch.float16).to(torch.bfloat16)
        assert oracle.half_to_bf16(h) == int(ref_h.view(torch.int16).item()) & 0xFFFF


def test_dequant_rejects_bad_layout():
    with pytest.raises(RuntimeError):
        oracle.dequant(np.zeros((2, 10), np.int8), np.zeros(2, np.uint16), np.zeros(2, np.uint16), 300, 128)
