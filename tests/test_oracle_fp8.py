"""Pins the oracle's number-format conversions against torch's library casts."""
import numpy as np
import torch

from oracle import fp8 as ofp8


def torch_e4m3(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x.astype(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_e4m3_decode_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    ours = ofp8.e4m3fn_to_f32(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(np.isnan(ours), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(ours[ok].view(np.uint32), ref[ok].view(np.uint32))


def test_e4m3_encode_every_bf16_pattern():
    x = ofp8.bf16_to_f32(np.arange(65536, dtype=np.uint32).astype(np.uint16))
    assert np.array_equal(ofp8.f32_to_e4m3fn(x), torch_e4m3(x))


def test_e4m3_encode_midpoints_ties_to_even():
    vals = ofp8.e4m3fn_to_f32(np.arange(0, 0x7F, dtype=np.uint8)).astype(np.float64)
    mids = (vals[:-1] + vals[1:]) / 2  # exact in fp32
    pts = np.concatenate([mids, -mids]).astype(np.float32)
    nudged = np.concatenate([np.nextafter(pts, np.float32(np.inf)), np.nextafter(pts, np.float32(-np.inf))])
    for arr in (pts, nudged, np.array([448, 464, 465, 480, 1e9, -1e9, np.inf, -np.inf], np.float32)):
        assert np.array_equal(ofp8.f32_to_e4m3fn(arr), torch_e4m3(arr))


def test_e4m3_encode_random_fp32():
    rng = np.random.default_rng(1)
    for scale in (1e-4, 1e-2, 1.0, 30.0, 448.0):
        x = (rng.standard_normal(200_000) * scale).astype(np.float32)
        assert np.array_equal(ofp8.f32_to_e4m3fn(x), torch_e4m3(x))


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(2)
    x = rng.standard_normal(100_000).astype(np.float32) * 10
    ties = ofp8.bf16_to_f32(rng.integers(0, 2**16, 1000, dtype=np.uint16)).view(np.uint32) | np.uint32(0x8000)
    x = np.concatenate([x, ties.view(np.float32)])
    x = x[np.isfinite(x)]
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ofp8.f32_to_bf16(x), ref)


def test_fp16_decode_matches_numpy_half():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = torch.from_numpy(bits.view(np.int16)).view(torch.float16).float().numpy()
    ours = ofp8.fp16_to_f32(bits)
    ok = ~np.isnan(ref)
    assert np.array_equal(ours[ok], ref[ok])
