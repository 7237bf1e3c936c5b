"""GPU parity of the 4-bit codec kernels against the oracle (bit-exact).

Each test prints the case it runs before touching the GPU.
"""
import json
import os

import numpy as np
import pytest
import torch

import oracle
from usaf_amd import quantization as Q

pytestmark = pytest.mark.gpu
KAT = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "q4_kat.json")))


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16).reshape(-1)


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16])
def test_cfg0_roundtrip_bit_exact(gpu_device, out_dtype):
    _say(f"cfg0 [768,2048] quantize+dequant {out_dtype}")
    g = torch.Generator().manual_seed(1234)
    w = (torch.randn(768, 2048, generator=g) * 0.02).half()
    p_o, s_o, z_o = oracle.quantize(w.float().numpy(), 128)
    p, s, z, shape = Q.quantize_4bit(w.to(gpu_device), 128)
    torch.cuda.synchronize()
    assert shape == w.shape and p.shape == (12288, 64) and p.dtype == torch.int8
    assert np.array_equal(p.cpu().numpy(), p_o), "codes differ"
    assert np.array_equal(_bits(s), s_o) and np.array_equal(_bits(z), z_o)
    d = Q.dequantize_4bit(p, s, z, shape, 128, out_dtype=out_dtype)
    torch.cuda.synchronize()
    ref = oracle.dequant(p_o, s_o, z_o, w.numel(), 128, out_dtype="bf16" if out_dtype == torch.bfloat16 else "f16")
    assert d.shape == w.shape and d.dtype == out_dtype
    assert np.array_equal(_bits(d), ref)


@pytest.mark.parametrize("shape,gs", [((3, 333), 128), ((7,), 128), ((5, 7), 3), ((1000,), 64),
                                      ((129,), 128), ((2, 255), 5), ((4099,), 128), ((64, 96), 256)])
@pytest.mark.parametrize("x_dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_ragged_shapes(gpu_device, shape, gs, x_dtype):
    _say(f"ragged shape={shape} gs={gs} x={x_dtype}")
    g = torch.Generator().manual_seed(99)
    w = (torch.randn(shape, generator=g) * 0.5).to(x_dtype)
    p_o, s_o, z_o = oracle.quantize(w.float().numpy().reshape(-1), gs)
    p, s, z, _ = Q.quantize_4bit(w.to(gpu_device), gs)
    torch.cuda.synchronize()
    assert np.array_equal(p.cpu().numpy(), p_o)
    assert np.array_equal(_bits(s), s_o) and np.array_equal(_bits(z), z_o)
    for od, tag in ((torch.float16, "f16"), (torch.bfloat16, "bf16")):
        d = Q.dequantize_4bit(p, s, z, w.shape, gs, out_dtype=od)
        torch.cuda.synchronize()
        assert np.array_equal(_bits(d), oracle.dequant(p_o, s_o, z_o, w.numel(), gs, out_dtype=tag))


@pytest.mark.parametrize("name", ["ramp", "pad_tail", "constant", "tiny", "odd_gs3"])
def test_quantize_kat(gpu_device, name):
    _say(f"quantize KAT {name}")
    k = next(k for k in KAT if k["name"] == name)
    p, s, z, _ = Q.quantize_4bit(torch.tensor(k["x"], dtype=torch.float32, device=gpu_device), k["group_size"])
    torch.cuda.synchronize()
    assert p.cpu().tolist() == k["packed"]
    assert _bits(s).tolist() == k["scale"] and _bits(z).tolist() == k["zero"]


@pytest.mark.parametrize("name", ["ramp", "constant", "odd_gs3_dequant_layout"])
def test_dequant_kat(gpu_device, name):
    _say(f"dequant KAT {name}")
    k = next(k for k in KAT if k["name"] == name)
    p = torch.tensor(k["packed"], dtype=torch.int8, device=gpu_device)
    s = torch.tensor(k["scale"], dtype=torch.int32).to(torch.int16).view(torch.float16).to(gpu_device)
    z = torch.tensor(k["zero"], dtype=torch.int32).to(torch.int16).view(torch.float16).to(gpu_device)
    d = Q.dequantize_4bit(p, s, z, torch.Size([len(k["dequant_f16"])]), k["group_size"])
    torch.cuda.synchronize()
    assert _bits(d).tolist() == k["dequant_f16"]


def test_double_rounding_kat(gpu_device):
    _say("double rounding KAT on the fast path (group 128)")
    cases = next(k for k in KAT if k["name"] == "double_rounding")["cases"]
    G = len(cases)
    codes = np.zeros((G, 128), np.uint8)
    s = np.zeros(G, np.uint16)
    z = np.zeros(G, np.uint16)
    for i, (q, sb, zb, _, _) in enumerate(cases):
        codes[i, :] = q
        s[i], z[i] = sb, zb
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).view(np.int8)
    d = Q.dequantize_4bit(torch.from_numpy(packed).to(gpu_device),
                          torch.from_numpy(s.view(np.int16)).view(torch.float16).to(gpu_device),
                          torch.from_numpy(z.view(np.int16)).view(torch.float16).to(gpu_device),
                          torch.Size([G * 128]), 128)
    torch.cuda.synchronize()
    got = _bits(d).reshape(G, 128)
    for i, c in enumerate(cases):
        assert np.all(got[i] == c[3]), f"case {i}: got {got[i][0]:#x}, two-rounding {c[3]:#x}, fma {c[4]:#x}"


def test_exhaustive_scales_fast_path(gpu_device):
    _say("every finite fp16 scale x every code, fast path")
    s_all = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    s_all = s_all[np.isfinite(s_all.view(np.float16))]
    G = s_all.size
    rng = np.random.default_rng(3)
    codes = rng.integers(0, 16, size=(G, 128), dtype=np.uint8)
    codes[:, :16] = np.arange(16, dtype=np.uint8)
    z = rng.standard_normal(G).astype(np.float16).view(np.uint16)
    z[:16] = [0x7C00, 0xFC00, 0x7E00, 0x0001, 0x8001, 0x03FF, 0, 0x8000, 0x7BFF, 0xFBFF, 1, 2, 3, 4, 5, 6]
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).view(np.int8)
    ref16 = oracle.dequant(packed, s_all, z, G * 128, 128)
    ref_bf = oracle.dequant(packed, s_all, z, G * 128, 128, out_dtype="bf16")
    pt = torch.from_numpy(packed).to(gpu_device)
    st = torch.from_numpy(s_all.view(np.int16)).view(torch.float16).to(gpu_device)
    zt = torch.from_numpy(z.view(np.int16)).view(torch.float16).to(gpu_device)
    for od, ref in ((torch.float16, ref16), (torch.bfloat16, ref_bf)):
        d = Q.dequantize_4bit(pt, st, zt, torch.Size([G * 128]), 128, out_dtype=od)
        torch.cuda.synchronize()
        got = _bits(d)
        if od == torch.float16:  # NaN payloads of fp16 arithmetic are not pinned; compare NaN-ness
            nan = np.isnan(ref.view(np.float16))
            assert np.array_equal(np.isnan(got.view(np.float16)), nan)
            assert np.array_equal(got[~nan], ref[~nan])
        else:
            assert np.array_equal(got, ref)


def test_misaligned_output_takes_generic_path(gpu_device):
    _say("misaligned output view")
    g = torch.Generator().manual_seed(11)
    w = torch.randn(4096, generator=g).half()
    p_o, s_o, z_o = oracle.quantize(w.float().numpy(), 128)
    p, s, z, _ = Q.quantize_4bit(w.to(gpu_device), 128)
    buf = torch.empty(4096 + 1, dtype=torch.float16, device=gpu_device)
    out = buf[1:]
    Q.dequantize_4bit(p, s, z, w.shape, 128, out=out)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(out), oracle.dequant(p_o, s_o, z_o, 4096, 128))


def test_full_layer_sampled_groups(gpu_device):
    # Qwen3-30B-A3B gate_up [128, 1536, 2048] quantized on the GPU: bit-exact on
    # 2048 random groups against the oracle run on those groups alone (the
    # codec is group-local, so a group's result does not depend on the rest).
    _say("full gate_up [128,1536,2048] sampled groups")
    torch.manual_seed(0)
    w = (torch.randn(128, 1536, 2048, device=gpu_device) * 0.02).half()
    p, s, z, shape = Q.quantize_4bit(w, 128)
    d = Q.dequantize_4bit(p, s, z, shape, 128, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    G = p.shape[0]
    rng = np.random.default_rng(0)
    idx = torch.from_numpy(np.sort(rng.choice(G, 2048, replace=False))).to(gpu_device)
    wg = w.reshape(G, 128)[idx].float().cpu().numpy()
    p_o, s_o, z_o = oracle.quantize(wg.reshape(-1), 128)
    assert np.array_equal(p[idx].cpu().numpy(), p_o)
    assert np.array_equal(_bits(s[idx]), s_o) and np.array_equal(_bits(z[idx]), z_o)
    ref = oracle.dequant(p_o, s_o, z_o, wg.size, 128, out_dtype="bf16")
    assert np.array_equal(_bits(d.reshape(G, 128)[idx]), ref)
    del w, d


def test_state_dict_wrappers(gpu_device):
    _say("quantize_state_dict / dequantize_state_dict")
    sd = {"a": torch.randn(300, 7), "b": torch.randn(10), "c": torch.tensor(3.0), "n": 5}
    qd = Q.quantize_state_dict(sd, group_size=128, min_size=256)
    assert isinstance(qd["a"], dict) and qd["a"]["group_size"] == 128
    assert qd["b"].dtype == torch.float16 and qd["c"].dtype == torch.float16 and qd["n"] == 5
    dd = Q.dequantize_state_dict(qd)
    torch.cuda.synchronize()
    p_o, s_o, z_o = oracle.quantize(sd["a"].float().numpy().reshape(-1), 128)
    assert np.array_equal(_bits(dd["a"]), oracle.dequant(p_o, s_o, z_o, 2100, 128))
    assert dd["a"].shape == (300, 7)


@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16])
def test_dequant_slices_jobs(gpu_device, out_dtype):
    """usaf_hip_dequant_q4_slices: job j dequantizes slice src[j] into arena slot
    dst[j] (natural order), bit-exact against the oracle's dequant of that slice;
    slots no job names keep their contents, jobs naming a slice or slot out of
    range are skipped."""
    from usaf_amd import _native as N
    _say(f"slice dequant jobs into an arena, {out_dtype}")
    E, rows, cols = 6, 64, 256
    slice_elems = rows * cols
    g = torch.Generator().manual_seed(31)
    w = (torch.randn(E, rows, cols, generator=g) * 0.02).half().to(gpu_device)
    p, s, z, shape = Q.quantize_4bit(w, 128)
    n_slots = 5
    arena = torch.full((n_slots, slice_elems), 7.0, dtype=out_dtype, device=gpu_device)
    src = torch.tensor([4, 0, 2, 9, 1], dtype=torch.int64)   # 9: past the tensor
    dst = torch.tensor([0, 3, 1, 2, 7], dtype=torch.int64)   # 7: past the arena
    src_d, dst_d = src.to(gpu_device), dst.to(gpu_device)
    N.call("usaf_hip_dequant_q4_slices", p.data_ptr(), s.data_ptr(), z.data_ptr(), p.shape[0], slice_elems,
           len(src), src_d.data_ptr(), dst_d.data_ptr(), n_slots, arena.data_ptr(), N.dtype_code(out_dtype),
           N.stream_ptr(gpu_device))
    torch.cuda.synchronize()
    pc, sc, zc = p.cpu().numpy(), _bits(s), _bits(z)
    gps = slice_elems // 128
    odt = "bf16" if out_dtype == torch.bfloat16 else "f16"
    filled = set()
    for e, d in zip(src.tolist(), dst.tolist()):
        if e >= E or d >= n_slots:
            continue
        ref = oracle.dequant(pc[e * gps:(e + 1) * gps], sc[e * gps:(e + 1) * gps], zc[e * gps:(e + 1) * gps],
                             slice_elems, 128, out_dtype=odt)
        assert np.array_equal(_bits(arena[d]), ref), (e, d)
        filled.add(d)
    for d in set(range(n_slots)) - filled:
        assert torch.all(arena[d] == 7.0), d


@pytest.mark.parametrize("w_rows,K,inter", [(384, 128, 0), (384, 256, 192), (256, 128, 128)])
def test_dequant_slices_frag_layout(gpu_device, w_rows, K, inter):
    """usaf_hip_dequant_q4_slices_frag: the dequant of each named expert in the
    fragment order of the slot GEMMs (padding rows zero), bit-exact against
    the oracle's dequant permuted by the layout map; jobs out of range skipped."""
    from usaf_amd import _native as N
    from usaf_amd.expert_cache import frag_chunk_index
    _say(f"fragment-order fill w_rows={w_rows} K={K} inter={inter}")
    E = 3
    g = torch.Generator().manual_seed(w_rows + K + inter)
    w = (torch.randn(E, w_rows, K, generator=g) * 0.02).half().to(gpu_device)
    p, s, z, shape = Q.quantize_4bit(w, 128)
    slot = int(N.load().usaf_hip_frag_slot_elems(w_rows, K, inter))
    n_slots = 3
    arena = torch.full((n_slots, slot), 7.0, dtype=torch.float16, device=gpu_device)
    src = torch.tensor([2, 0, 5], dtype=torch.int64, device=gpu_device)  # 5: past the tensor
    dst = torch.tensor([0, 2, 1], dtype=torch.int64, device=gpu_device)
    N.call("usaf_hip_dequant_q4_slices_frag", p.data_ptr(), s.data_ptr(), z.data_ptr(), E, w_rows, K, inter, 3,
           src.data_ptr(), dst.data_ptr(), n_slots, arena.data_ptr(), N.F16, N.stream_ptr(gpu_device))
    torch.cuda.synchronize()
    idx = frag_chunk_index(w_rows, K, inter)
    ref_all = oracle.dequant(p.cpu().numpy(), _bits(s), _bits(z), E * w_rows * K, 128).reshape(E, -1, 8)
    for e, d in ((2, 0), (0, 2)):
        got = _bits(arena[d]).reshape(-1, 8)
        keep = (idx >= 0).numpy()
        assert np.array_equal(got[keep], ref_all[e][idx[idx >= 0].numpy()])
        assert np.all(got[~keep] == 0)
    assert torch.all(arena[1] == 7.0)
