"""Pins the CPU oracle (oracle/dotcache_oracle.py) by checks other than a
retyping of its formulas:

* the reference's own tests for this path, restated against the oracle
  (reference tests/test_pack_unpack.py, test_m0_quant.py, test_page_format.py,
  test_score_reference.py, test_mix_reference.py, test_attention_vs_dense.py,
  test_escape_mode.py, test_model_kv_cache.py:45-47);
* hand-derived known answers: round-half-even ties, exact scales, constant
  groups whose 1e-8 scale underflows fp16, clipping, the fp32-vs-fp16 scale
  used for codes, int8 escape rounding;
* an independent packer (Python big integers) for every code width;
* brute force: streaming score / mix / decode against dense dequantised
  attention computed in float64.
"""
from fractions import Fraction

import numpy as np
import pytest

from oracle import dotcache_oracle as O


def _bigint_pack(codes, bits):
    """Independent packer: concatenate symbols into one Python int."""
    codes = np.asarray(codes, dtype=np.int64)
    n = codes.shape[-1]
    nw = (n * bits + 31) // 32
    out = np.zeros(codes.shape[:-1] + (nw,), dtype=np.uint32)
    for idx in np.ndindex(codes.shape[:-1]):
        acc = 0
        for k, c in enumerate(codes[idx]):
            acc |= int(c) << (k * bits)
        for w in range(nw):
            out[idx + (w,)] = (acc >> (32 * w)) & 0xFFFFFFFF
    return out


# ---- packing: reference tests/test_pack_unpack.py ------------------------

def test_pack_unpack_roundtrip_4bit():
    codes = np.array([[0, 1, 2, 3, 4, 5, 6, 15]], dtype=np.uint8)
    packed = O.pack_bits(codes, 4)
    np.testing.assert_array_equal(O.unpack_bits(packed, 4, 8), codes)
    assert packed[0, 0] == 0xF6543210  # known answer: nibble k at bits 4k


def test_pack_unpack_roundtrip_2bit():
    codes = np.array([[0, 1, 2, 3, 0, 1, 2, 3]], dtype=np.uint8)
    np.testing.assert_array_equal(O.unpack_bits(O.pack_bits(codes, 2), 2, 8), codes)


def test_pack_unpack_handles_partial_word():
    codes = np.arange(24, dtype=np.uint8)[None, :] % 4
    packed = O.pack_bits(codes, 2)
    assert packed.shape[-1] == O.words_per_group(24, 2)
    np.testing.assert_array_equal(O.unpack_bits(packed, 2, 24), codes)


def test_pack_unpack_roundtrip_3bit_with_spill():
    codes = (np.arange(32, dtype=np.uint8)[None, :] % 8).astype(np.uint8)
    packed = O.pack_bits(codes, 3)
    assert packed.shape[-1] == O.words_per_group(32, 3)
    np.testing.assert_array_equal(O.unpack_bits(packed, 3, 32), codes)


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 8])
@pytest.mark.parametrize("n", [8, 24, 32, 64])
def test_pack_matches_independent_bigint_packer(bits, n):
    rng = np.random.default_rng(bits * 100 + n)
    codes = rng.integers(0, 1 << bits, size=(3, 2, n), dtype=np.uint8)
    np.testing.assert_array_equal(O.pack_bits(codes, bits), _bigint_pack(codes, bits))
    np.testing.assert_array_equal(O.unpack_bits(O.pack_bits(codes, bits), bits, n), codes)


def test_pack_rejects_out_of_range_codes():
    with pytest.raises(ValueError):
        O.pack_bits(np.array([[16]], dtype=np.uint8), 4)


def test_words_per_group_known_answers():
    assert O.words_per_group(32, 4) == 4
    assert O.words_per_group(32, 8) == 8
    assert O.words_per_group(64, 8) == 16
    assert O.words_per_group(32, 3) == 3
    with pytest.raises(ValueError):
        O.words_per_group(0, 4)


# ---- page format: reference tests/test_page_format.py ---------------------

def test_build_payload_group_major_matches_per_group_pack_for_3bit():
    codes = (np.arange(2 * 4 * 32, dtype=np.uint8).reshape(2, 4, 32) % 8).astype(np.uint8)
    payload = O.build_payload(codes, 3, "group_major")
    expected = np.stack([_bigint_pack(codes[:, g, :], 3) for g in range(4)], axis=0)
    np.testing.assert_array_equal(payload, expected)


def test_header_json_roundtrip_and_sorted_keys():
    page = O.encode_page(np.ones((2, 32), np.float32), head_dim=32, group_size=32, bits=4, kind="K")
    js = page.header.to_json()
    import json

    d = json.loads(js)
    assert list(d.keys()) == sorted(d.keys())
    assert len(d) == 20
    assert d["mode_default"] == "M0" and d["words_per_group"] == 4 and d["padded_head_dim"] == 32


# ---- M0 quantisation: reference tests/test_m0_quant.py + known answers -----

def test_affine_quantization_shapes_and_error():
    rng = np.random.default_rng(0)
    values = rng.normal(size=(4, 48)).astype(np.float32)
    codes, scales, bias, phd = O.quantize_tensor(values, group_size=32, bits=4, scheme="affine")
    decoded = O.dequantize_groups(codes, scales=scales, bias=bias, bits=4, scheme="affine").reshape(4, phd)[:, :48]
    assert codes.shape == (4, 2, 32) and scales.shape == (4, 2) and bias.shape == (4, 2) and phd == 64
    assert np.max(np.abs(values - decoded)) < 0.35


def test_symmetric_quantization_roundtrip_is_reasonable():
    rng = np.random.default_rng(1)
    values = rng.normal(size=(3, 32)).astype(np.float32)
    codes, scales, bias, phd = O.quantize_tensor(values, group_size=32, bits=4, scheme="symmetric")
    decoded = O.dequantize_groups(codes, scales=scales, bias=bias, bits=4, scheme="symmetric").reshape(3, phd)
    assert bias is None
    assert np.max(np.abs(values - decoded)) < 0.4


def test_affine_quantization_3bit_roundtrip_is_reasonable():
    rng = np.random.default_rng(2)
    values = rng.normal(size=(4, 48)).astype(np.float32)
    codes, scales, bias, phd = O.quantize_tensor(values, group_size=32, bits=3, scheme="affine")
    decoded = O.dequantize_groups(codes, scales=scales, bias=bias, bits=3, scheme="affine").reshape(4, phd)[:, :48]
    assert np.max(np.abs(values - decoded)) < 0.8


def test_affine_known_answer_half_even_ties():
    # min 0, max 15 -> scale exactly 1: codes = round-half-even(x)
    x = np.array([[0, 15, 2.5, 3.5, 0.5, 1.5, 14.5, 7.25]], np.float32)
    codes, scales, bias, _ = O.quantize_tensor(x, group_size=8, bits=4, scheme="affine")
    np.testing.assert_array_equal(codes[0, 0], [0, 15, 2, 4, 0, 2, 14, 7])
    assert scales[0, 0] == 1.0 and bias[0, 0] == 0.0


def test_affine_known_answer_negative_offset():
    x = np.array([[-3, 12, -2.5, 0.0, 4.5]], np.float32)  # scale 1, bias -3 -> rint(x + 3)
    codes, scales, bias, _ = O.quantize_tensor(x, group_size=5, bits=4, scheme="affine")
    np.testing.assert_array_equal(codes[0, 0], [0, 15, 0, 3, 8])  # 0.5 -> 0, 7.5 -> 8
    assert bias[0, 0] == -3.0


def test_constant_group_scale_underflows_fp16():
    x = np.full((1, 32), 5.0, np.float32)
    page = O.encode_page(x, head_dim=32, group_size=32, bits=4, kind="K")
    assert page.scales[0, 0] == 0.0  # fp32 1e-8 is below half the smallest fp16 subnormal
    assert page.bias[0, 0] == np.float16(5.0)
    assert np.all(O.unpack_bits(page.payload[0], 4, 32) == 0)


def test_scale_is_correctly_rounded_fp32_division():
    x = np.zeros((1, 32), np.float32)
    x[0, 1] = 1.0  # max - min = 1 -> scale = fp32(1/15)
    _, scales, _, _ = O.quantize_tensor(x, group_size=32, bits=4, scheme="affine")
    # nearest fp32 to 1/15, found by exhaustive neighbour search on exact rationals
    cand = np.float32(1 / 15)
    best = min((cand, np.nextafter(cand, np.float32(1)), np.nextafter(cand, np.float32(0))),
               key=lambda f: abs(Fraction(float(f)) - Fraction(1, 15)))
    assert scales[0, 0] == best


def test_codes_use_fp32_scale_not_fp16_scale():
    # scale = 1.1/15 in fp32; x chosen so x/scale_fp32 and x/scale_fp16 round to different codes
    x = np.zeros((1, 32), np.float32)
    x[0, 1] = np.float32(1.1)
    s32 = np.float32(np.float32(1.1) / np.float32(15))
    s16 = np.float32(np.float16(s32))
    found = None
    for k in range(1, 15):
        for frac in np.linspace(-0.49, 0.49, 393):
            v = np.float32((k + 0.5 + frac * 0.01) * s32)
            if np.rint(v / s32) != np.rint(v / s16):
                found = v
                break
        if found is not None:
            break
    assert found is not None
    x[0, 2] = found
    codes, scales, _, _ = O.quantize_tensor(x, group_size=32, bits=4, scheme="affine")
    assert scales[0, 0] == s32
    assert codes[0, 0, 2] == np.rint(found / s32)
    page = O.encode_page(x, head_dim=32, group_size=32, bits=4, kind="K")
    assert page.scales[0, 0] == np.float16(s32)


def test_symmetric_known_answers():
    x = np.array([[-7, 7, 0.5, -0.5, 1.5, -2.5, 6.5, 3.0]], np.float32)  # scale 1
    codes, scales, bias, _ = O.quantize_tensor(x, group_size=8, bits=4, scheme="symmetric")
    np.testing.assert_array_equal(codes[0, 0], [0, 14, 7, 7, 9, 5, 13, 10])
    assert scales[0, 0] == 1.0 and bias is None
    x8 = np.array([[-127, 127, 0.5, 1.5, -126.5, 3]], np.float32)
    codes8, s8, _, _ = O.quantize_tensor(x8, group_size=6, bits=8, scheme="symmetric")
    np.testing.assert_array_equal(codes8[0, 0], [0, 254, 127, 129, 1, 130])


def test_symmetric_clips_at_qmax():
    # |x| max 7 with a larger negative pushed down: codes stay in [0, 14]
    x = np.array([[7.0, -7.0, 6.9, -6.9]], np.float32)
    codes, _, _, _ = O.quantize_tensor(x, group_size=4, bits=4, scheme="symmetric")
    assert codes.min() >= 0 and codes.max() <= 14


def test_padding_channels_join_min_max():
    x = np.full((1, 40), 3.0, np.float32)  # padded to 64 with zeros
    codes, scales, bias, phd = O.quantize_tensor(x, group_size=32, bits=4, scheme="affine")
    assert phd == 64
    assert bias[0, 1] == 0.0 and scales[0, 1] == np.float32(np.float32(3.0) / np.float32(15))


# ---- M3 escape: reference tests/test_escape_mode.py -------------------------

def test_escape_page_roundtrip_fp16():
    rng = np.random.default_rng(5)
    values = rng.normal(size=(3, 32)).astype(np.float32)
    page = O.encode_page(values, head_dim=32, group_size=32, bits=4, kind="K", mode="M3")
    assert page.escape_payload.dtype == np.float16
    np.testing.assert_array_equal(page.escape_payload, values.astype(np.float16))
    np.testing.assert_allclose(O.decode_escape_payload(page.escape_payload, head_dim=32), values, atol=1e-3, rtol=1e-3)


def test_escape_int8_known_answer():
    x = np.array([[127.0, -63.5, 0.0, 62.5]], np.float32)
    q, s = O.encode_escape_storage(x, "int8")
    assert s[0] == np.float16(1.0)
    np.testing.assert_array_equal(q[0], [127, -64, 0, 62])


def test_escape_page_int8_roundtrip():
    rng = np.random.default_rng(15)
    values = rng.normal(size=(5, 32)).astype(np.float32)
    page = O.encode_page(values, head_dim=32, group_size=32, bits=4, kind="K", mode="M3", escape_dtype="int8")
    decoded = O.decode_escape_payload(page.escape_payload, head_dim=32, scales=page.escape_scales)
    np.testing.assert_allclose(decoded, values, atol=0.08, rtol=0.08)


# ---- read path: reference test_score/mix_reference, test_attention_vs_dense ----

def _dense64(page):
    return O.decode_page(page).astype(np.float64)


@pytest.mark.parametrize("scheme", ["affine", "symmetric"])
@pytest.mark.parametrize("bits", [2, 3, 4, 8])
def test_score_page_matches_explicit_dequantized_baseline(scheme, bits):
    rng = np.random.default_rng(2)
    keys = rng.normal(size=(6, 48)).astype(np.float32)
    query = rng.normal(size=(48,)).astype(np.float32)
    page = O.encode_page(keys, head_dim=48, group_size=32, bits=bits, kind="K", scheme=scheme)
    streaming = O.score_page_ref(query, page)
    assert page.full_page_decode_calls == 0
    np.testing.assert_allclose(streaming, _dense64(page) @ query.astype(np.float64), atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("scheme", ["affine", "symmetric"])
def test_mix_page_matches_explicit_dequantized_baseline(scheme):
    rng = np.random.default_rng(3)
    values = rng.normal(size=(7, 48)).astype(np.float32)
    attn = O.softmax(rng.normal(size=(7,)).astype(np.float32))
    page = O.encode_page(values, head_dim=48, group_size=32, bits=4, kind="V", scheme=scheme)
    mixed = O.mix_page_ref(attn, page)
    assert page.full_page_decode_calls == 0
    np.testing.assert_allclose(mixed, attn.astype(np.float64) @ _dense64(page), atol=1e-5, rtol=1e-5)


def test_escape_page_score_and_mix_behave_like_dense_storage():
    rng = np.random.default_rng(6)
    keys = rng.normal(size=(4, 32)).astype(np.float32)
    values = rng.normal(size=(4, 32)).astype(np.float32)
    query = rng.normal(size=(32,)).astype(np.float32)
    attn = O.softmax(rng.normal(size=(4,)).astype(np.float32))
    kp = O.encode_page(keys, head_dim=32, group_size=32, bits=4, kind="K", mode="M3")
    vp = O.encode_page(values, head_dim=32, group_size=32, bits=4, kind="V", mode="M3")
    np.testing.assert_allclose(O.score_page_ref(query, kp), O.explicit_dequantized_score(query, kp), atol=1e-3, rtol=1e-3)
    np.testing.assert_allclose(O.score_page_ref(query, kp), keys.astype(np.float16).astype(np.float64) @ query, atol=1e-5)
    np.testing.assert_allclose(O.mix_page_ref(attn, vp), attn @ values, atol=1e-3, rtol=1e-3)


def test_softmax_known_answers_and_invariants():
    w = O.softmax(np.array([0.0, np.log(2.0)], np.float32))
    np.testing.assert_allclose(w, [1 / 3, 2 / 3], rtol=1e-6)
    x = np.random.default_rng(9).normal(size=50).astype(np.float32)
    np.testing.assert_allclose(O.softmax(x), O.softmax(x + 100.0), rtol=1e-5, atol=1e-7)
    assert abs(float(O.softmax(x).sum()) - 1.0) < 1e-6


def test_decode_step_matches_dense_attention_over_pages():
    rng = np.random.default_rng(4)
    hd, n = 64, 150
    keys = rng.normal(size=(n, hd)).astype(np.float32)
    values = rng.normal(size=(n, hd)).astype(np.float32)
    q = rng.normal(size=(hd,)).astype(np.float32)
    kp = O.encode_pages(keys, tokens_per_page=64, head_dim=hd, group_size=32, bits=4, kind="K")
    vp = O.encode_pages(values, tokens_per_page=64, head_dim=hd, group_size=32, bits=4, kind="V", scheme="symmetric")
    assert [p.header.token_count for p in kp] == [64, 64, 22]
    logits, weights, out = O.decode_step(q, kp, vp)
    K = np.concatenate([_dense64(p) for p in kp])
    V = np.concatenate([_dense64(p) for p in vp])
    ref_logits = K @ q.astype(np.float64)
    e = np.exp(ref_logits - ref_logits.max())
    ref_w = e / e.sum()
    np.testing.assert_allclose(logits, ref_logits, atol=1e-4)
    np.testing.assert_allclose(weights, ref_w, atol=1e-6)
    np.testing.assert_allclose(out, ref_w @ V, atol=1e-5)


def test_decode_step_rejects_mismatched_pages():
    p = O.encode_page(np.ones((2, 32), np.float32), head_dim=32, group_size=32, bits=4, kind="K")
    with pytest.raises(ValueError):
        O.decode_step(np.ones(32, np.float32), [p], [])
    with pytest.raises(ValueError):
        O.decode_step(np.ones(32, np.float32), [], [])


def test_default_q_head_to_kv_head_maps_gqa_groups():
    np.testing.assert_array_equal(O.default_q_head_to_kv_head(8, 2), [0, 0, 0, 0, 1, 1, 1, 1])
    np.testing.assert_array_equal(O.default_q_head_to_kv_head(28, 4)[:8], [0] * 7 + [1])


def test_page_device_nbytes_matches_survey_byte_counts():
    # C3 V page: hd 128, sym 4-bit g32, 64 tokens -> 4096 B codes + 512 B fp16 scales
    v = np.random.default_rng(1).normal(size=(64, 128)).astype(np.float32)
    vp = O.encode_page(v, head_dim=128, group_size=32, bits=4, kind="V", scheme="symmetric")
    assert O.page_device_nbytes(vp) == 4608
    kp = O.encode_page(v, head_dim=128, group_size=32, bits=4, kind="K", mode="M3")
    assert O.page_device_nbytes(kp) == 16384
    ap = O.encode_page(v, head_dim=128, group_size=32, bits=4, kind="K")
    assert O.page_device_nbytes(ap) == 4096 + 512 + 512
