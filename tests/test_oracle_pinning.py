"""Pins of the CPU oracle (oracle/psq_oracle.c + oracle/__init__.py), no GPU.

Each oracle function is checked against something it does not share code with: the reference's
own construction and known answers (powershard/operations.py:72-93, tests/test_portable.py:50-72,
tests/test_fp16_safe.py:85,171-174), library routines (numpy int64 matmul, float64 matmul, torch
casts to bfloat16 / float8_e4m3fn, numpy float16), closed forms, and brute force on tiny inputs.
Several tests plant a plausible mistake in a copy of the computation to show the check catches it.
"""
import numpy as np
import pytest
import torch

import oracle

GROUPS = [4, 16, 64, 256, 1024]


def sylvester(g):
    h = np.array([[1.0]])
    while h.shape[0] < g:
        h = np.block([[h, h], [h, -h]])
    return h / np.sqrt(g)


# ------------------------------------------------------------------- Hadamard
@pytest.mark.parametrize("g", GROUPS)
def test_hadamard_closed_form_matches_kron_construction(g):
    """closed form == Kronecker powers of H4 (powershard/operations.py:72-81)."""
    h = oracle.regular_hadamard(g).double().numpy()
    assert np.array_equal(h, oracle.regular_hadamard_kron(g))


@pytest.mark.parametrize("g", GROUPS)
def test_hadamard_orthonormal_exactly(g):
    """H @ H.T == I with zero tolerance (tests/test_portable.py:51-52) and H symmetric."""
    h = oracle.regular_hadamard(g)
    assert torch.equal(h @ h.T, torch.eye(g))
    assert torch.equal(h, h.T)


def test_hadamard_is_not_sylvester():
    """The reference's regular H is not the Sylvester matrix (operations.py:74): a transform
    built on Sylvester would fail the other pins."""
    for g in (16, 256):
        assert not np.allclose(oracle.regular_hadamard(g).double().numpy(), sylvester(g))


@pytest.mark.parametrize("g", [0, 2, 3, 8, 32, 128, 512])
def test_hadamard_rejects_non_powers_of_4(g):
    with pytest.raises(ValueError):
        oracle.regular_hadamard(g)


# ------------------------------------------------------------------ rotation
@pytest.mark.parametrize("g", GROUPS)
def test_rotation_matches_dense_product(g):
    """fast transform == x @ H in float64 within fp32 rounding."""
    x = (torch.randn(7, 2048, generator=torch.Generator().manual_seed(g)) * 3).to(torch.bfloat16)
    got = oracle.rotate_rows(x, g).double()
    h = torch.from_numpy(oracle.regular_hadamard_kron(g))
    ref = (x.double().reshape(7, -1, g) @ h).reshape(7, 2048)
    assert (got - ref).abs().max().item() <= 1e-6 * ref.abs().max().item()


@pytest.mark.parametrize("g", GROUPS)
def test_rotation_exact_on_small_integers(g):
    """Integer inputs keep every partial sum exact: the fast transform equals the dense product."""
    x = torch.randint(-8, 9, (5, 2048), generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    got = oracle.rotate_rows(x, g).double()
    h = torch.from_numpy(oracle.regular_hadamard_kron(g))
    ref = (x.double().reshape(5, -1, g) @ h).reshape(5, 2048)
    assert torch.equal(got, ref)
    # planted mistake: a Sylvester-based rotation differs
    hs = torch.from_numpy(sylvester(g))
    wrong = (x.double().reshape(5, -1, g) @ hs).reshape(5, 2048)
    assert not torch.equal(got, wrong)


def test_rotation_unit_vectors_give_hadamard_rows():
    """Rotating e_j gives row j of H: every entry +-2^-k, signs from the closed form."""
    g = 256
    x = torch.zeros(g, g, dtype=torch.bfloat16)
    x[torch.arange(g), torch.arange(g)] = 1
    assert torch.equal(oracle.rotate_rows(x, g), oracle.regular_hadamard(g))


# -------------------------------------------------------------- int8 quantize
def test_quantize_known_rows_without_rotation():
    """x = q_true * 2^-e with max|q_true| = 127 -> codes == q_true, scale == 2^-e exactly."""
    g = torch.Generator().manual_seed(3)
    q_true = torch.randint(-127, 128, (16, 512), generator=g)
    q_true[:, 7] = 127
    e = torch.arange(16) - 8
    x = (q_true.double() * torch.pow(2.0, -e.double())[:, None]).to(torch.bfloat16)
    assert torch.equal(x.double(), q_true.double() * torch.pow(2.0, -e.double())[:, None])
    q, s = oracle.quantize_rows_i8(x)
    assert torch.equal(q.long(), q_true)
    assert torch.equal(s.double(), torch.pow(2.0, -e.double()))


def test_quantize_ties_round_to_even():
    """scale 1 (absmax 127): 2.5 -> 2, 3.5 -> 4, -2.5 -> -2, 0.5 -> 0, 1.5 -> 2."""
    x = torch.tensor([[127.0, 2.5, 3.5, -2.5, 0.5, 1.5, -0.5, 126.5] + [0.0] * 8], dtype=torch.bfloat16)
    q, s = oracle.quantize_rows_i8(x)
    assert s.item() == 1.0
    assert q[0, :8].tolist() == [127, 2, 4, -2, 0, 2, 0, 126]


def test_quantize_rotated_unit_vector():
    """x = c e_j in one group: rotation spreads it to +-c/16, so every code is +-127 with the
    signs of row j of H, and the scale is (c/16)/127."""
    g, c, j = 256, 3.0, 37
    x = torch.zeros(1, g, dtype=torch.bfloat16)
    x[0, j] = c
    q, s = oracle.quantize_rows_i8(x, g)
    sign = torch.sign(oracle.regular_hadamard(g)[j])
    assert torch.equal(q[0].float(), 127 * sign)
    # the unnormalized transform maps c e_j to +-c, so s = (c / 127) * 2^-4 in fp32 (= (c/16) / 127)
    assert s.item() == np.float32(np.float32(np.float32(c) / np.float32(127)) * np.float32(2.0 ** -4))


def test_quantize_zero_row_and_invariants():
    x = torch.randn(64, 1024, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    x[5] = 0
    for g in (0, 256):
        q, s = oracle.quantize_rows_i8(x, g)
        assert s[5].item() == 1.0 and int(q[5].abs().sum()) == 0
        nz = torch.arange(64) != 5
        assert int(q.abs().max()) <= 127
        assert torch.all(q[nz].abs().amax(1) == 127)
        u = oracle.rotate_rows(x, g) if g else x.float()
        assert torch.all((u[nz] - q[nz].float() * s[nz, None]).abs() <= s[nz, None] * 0.5001)


def test_quantize_static_scale_saturates():
    x = torch.tensor([[1000.0, -1000.0, 0.25, 0.0] + [0.0] * 12], dtype=torch.bfloat16)
    q, s = oracle.quantize_rows_i8(x, static_scale=0.5)
    assert s.item() == 0.5 and q[0, :4].tolist() == [127, -127, 0, 0]


# ------------------------------------------------------------------ codecs
def test_e4m3_decode_exhaustive_vs_torch():
    codes = torch.arange(256, dtype=torch.uint8)
    ref = codes.view(torch.float8_e4m3fn).float()
    got = torch.tensor([oracle.lib().psq_or_e4m3_to_f32(int(c)) for c in codes])
    both_nan = torch.isnan(ref) & torch.isnan(got)
    assert torch.all((ref == got) | both_nan)


def test_e4m3_encode_vs_torch():
    """Every finite e4m3 value, every midpoint and nudges around them, plus random values:
    round-to-nearest-even == torch's cast (inside +-448, where both saturate identically)."""
    vals = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    vals = vals[torch.isfinite(vals)].unique()
    mids = (vals[1:] + vals[:-1]) / 2
    nudge = torch.cat([mids * (1 + 2.0 ** -20), mids * (1 - 2.0 ** -20)])
    rnd = torch.randn(20000, generator=torch.Generator().manual_seed(4)) * 100
    x = torch.cat([vals, mids, nudge, rnd]).clamp(-448, 448)
    ref = x.to(torch.float8_e4m3fn).view(torch.uint8)
    got = torch.tensor([oracle.lib().psq_or_f32_to_e4m3(float(v)) for v in x], dtype=torch.uint8)
    # torch keeps the sign of zero; so does the oracle
    assert torch.equal(got, ref)


def test_bf16_and_f16_encoders_vs_library_casts():
    g = torch.Generator().manual_seed(5)
    x = torch.cat([torch.randn(20000, generator=g) * torch.pow(10.0, torch.randint(-30, 30, (20000,), generator=g)),
                   torch.tensor([0.0, -0.0, 65504.0, 65520.0, 65519.99, 6e-8, 3e-8, 1e-40, 3.4e38])])
    got_b = torch.tensor([oracle.lib().psq_or_f32_to_bf16(float(v)) for v in x], dtype=torch.int32)
    ref_b = x.to(torch.bfloat16).view(torch.int16).to(torch.int32) & 0xFFFF
    assert torch.equal(got_b, ref_b)
    xs = x[x.abs() < 6e4]
    got_h = np.array([oracle.lib().psq_or_f32_to_f16(float(v)) for v in xs], dtype=np.uint16)
    ref_h = xs.numpy().astype(np.float16).view(np.uint16)
    assert np.array_equal(got_h, ref_h)


# ------------------------------------------------------------------- GEMMs
def test_gemm_i8_matches_numpy_int64():
    g = torch.Generator().manual_seed(6)
    a = torch.randint(-127, 128, (37, 640), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (53, 640), generator=g, dtype=torch.int8)
    ref = a.numpy().astype(np.int64) @ w.numpy().astype(np.int64).T
    assert np.array_equal(oracle.gemm_i8_i32(a, w).numpy().astype(np.int64), ref)
    rows = [5, 0, 36]
    assert np.array_equal(oracle.gemm_i8_i32(a, w, rows).numpy().astype(np.int64), ref[rows])


def test_gemm_i8_extremes_do_not_overflow():
    a = torch.full((2, 13824), -127, dtype=torch.int8)
    w = torch.full((3, 13824), -127, dtype=torch.int8)
    assert int(oracle.gemm_i8_i32(a, w)[0, 0]) == 127 * 127 * 13824


def test_epilogue_within_one_ulp_of_float64():
    g = torch.Generator().manual_seed(7)
    c = torch.randint(-2 ** 26, 2 ** 26, (64, 96), generator=g, dtype=torch.int32)
    sa, sw = torch.rand(64, generator=g) * 1e-2, torch.rand(96, generator=g) * 1e-3
    b = torch.randn(96, generator=g).to(torch.bfloat16)
    y = oracle.epilogue_i32(c, sa, sw, b, out_dtype=torch.float32).double()
    prod = c.double() * (sa.double()[:, None] * sw.double()[None, :])
    ref = prod + b.double()[None, :]
    # int32 -> fp32 conversion, the scale product and the fma each round once
    assert torch.all((y - ref).abs() <= (prod.abs() + b.double().abs()[None, :]) * 2.0 ** -22)
    yb = oracle.epilogue_i32(c, sa, sw, b, out_dtype=torch.bfloat16)
    assert torch.equal(yb, y.float().to(torch.bfloat16))   # bf16 output = RNE of the fp32 value


def test_gemm_fp8_matches_float64_matmul():
    g = torch.Generator().manual_seed(8)
    a = (torch.randn(21, 256, generator=g) * 50).clamp(-448, 448).to(torch.float8_e4m3fn)
    w = (torch.randn(19, 256, generator=g) * 50).clamp(-448, 448).to(torch.float8_e4m3fn)
    sa, sw = torch.rand(21, generator=g), torch.tensor(0.01)
    y = oracle.gemm_fp8(a.view(torch.uint8), sa, w.view(torch.uint8), sw, None, out_dtype=torch.float32)
    exact = a.double() @ w.double().T
    ref = (exact.float().double() * (sa.double()[:, None] * 0.01)).float()
    assert torch.allclose(y, ref, rtol=2e-7, atol=0)


def test_gemm_fp8_e5m2_weights_match_float64_matmul():
    """e4m3 activations x e5m2 weights: the double sum of the torch-decoded operands."""
    g = torch.Generator().manual_seed(18)
    a = (torch.randn(17, 256, generator=g) * 50).clamp(-448, 448).to(torch.float8_e4m3fn)
    w = (torch.randn(23, 256, generator=g) * 3000).clamp(-57344, 57344).to(torch.float8_e5m2)
    sa, sw = torch.rand(17, generator=g), torch.rand(23, generator=g) * 1e-4
    y = oracle.gemm_fp8(a, sa, w, sw, None, out_dtype=torch.float32)
    exact = a.double() @ w.double().T
    ref = (exact.float().double() * (sa.double()[:, None] * sw.double()[None, :].float().double())).float()
    assert torch.allclose(y, ref, rtol=2e-7, atol=0)
    # the weights' format matters: read as e4m3 the same bytes give another product
    y43 = oracle.gemm_fp8(a, sa, w.view(torch.uint8), sw, None, out_dtype=torch.float32, w_e5m2=False)
    assert not torch.allclose(y43, y)


def test_e5m2_decode_exhaustive():
    """The oracle's e5m2 decode (written from the format's definition) is torch's on all 256 codes."""
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    got = oracle.e5m2_to_f32(codes)
    ref = codes.view(torch.float8_e5m2).float()
    assert torch.equal(torch.isnan(got), torch.isnan(ref))
    ok = ~torch.isnan(ref)
    assert torch.equal(got[ok], ref[ok])
    assert torch.isinf(ref).sum() == 2 and torch.isnan(ref).sum() == 6
    assert got[0x01] == 2.0 ** -16 and got[0x7B] == 57344.0


@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_dequant_e5m2_matches_torch_decode(per_row, out_dtype):
    """round_out(e5m2(q) * s): torch's float8_e5m2 decode times the fp32 scale, then torch's cast."""
    g = torch.Generator().manual_seed(43)
    codes = torch.randint(0, 256, (29, 80), generator=g, dtype=torch.uint8)
    codes[(codes & 0x7C) == 0x7C] = 0x7B          # finite codes only
    s = torch.rand(29, generator=g) * 1e-2 + 1e-4 if per_row else torch.tensor(2.7e-3)
    got = oracle.dequant_fp8(codes.view(torch.float8_e5m2), s, out_dtype)
    ref = (codes.view(torch.float8_e5m2).float() * (s[:, None] if per_row else s)).to(out_dtype)
    assert torch.equal(got.view(torch.int16) if out_dtype != torch.float32 else got,
                       ref.view(torch.int16) if out_dtype != torch.float32 else ref)


def test_gemm_wonly_matches_float64_matmul():
    g = torch.Generator().manual_seed(9)
    x = torch.randn(11, 384, generator=g).to(torch.bfloat16)
    wd = (torch.randn(13, 384, generator=g) * 0.02).to(torch.bfloat16)
    b = torch.randn(13, generator=g).to(torch.bfloat16)
    y = oracle.gemm_wonly(x, wd, None, b, out_dtype=torch.float32).double()
    ref = x.double() @ wd.double().T + b.double()
    assert torch.allclose(y, ref, rtol=1e-6, atol=1e-6)


# ---------------------------------------------------------------- weights
def test_uint4_pack_round_trip_and_error_bound():
    g = torch.Generator().manual_seed(10)
    w = torch.randn(40, 512, generator=g) * 0.05
    wq, s, z = oracle.quantize_weight_uint4(w, 128)
    assert wq.dtype == torch.uint8 and wq.shape == (40, 256) and s.shape == (40, 4)
    # nibble order: low nibble = even k
    lo, hi = wq & 15, wq >> 4
    deq = oracle.dequant_uint4(wq, s, z, 128, out_dtype=torch.float32)
    q = torch.stack([lo, hi], -1).reshape(40, 512).float()
    manual = (q - z.float().repeat_interleave(128, 1)) * s.float().repeat_interleave(128, 1)
    assert torch.equal(deq, manual)
    err = (deq - w).abs()
    assert torch.all(err <= 0.51 * s.float().repeat_interleave(128, 1) + 1e-6)


def test_dequant_i8_rows_matches_reference_formula():
    """FWHT-based ConvRot inverse == dequantize_rows' dense matmul (operations.py:84-93) within
    fp32 summation order; case of tests/test_portable.py:53-60 (seed 5, [13, 512], scale*1e-3)."""
    gen = torch.Generator().manual_seed(5)
    q = torch.randint(-100, 100, (13, 512), generator=gen, dtype=torch.int8)
    scale = torch.rand((13, 1), generator=gen) * .001
    got = oracle.dequant_i8_rows(q, scale, 256, out_dtype=torch.float32)
    ref = oracle.dequantize_rows(q, scale, True, 256, torch.float32)
    torch.testing.assert_close(got, ref, rtol=1e-6, atol=1e-6 * ref.abs().max().item())
    got16 = oracle.dequant_i8_rows(q, scale, 256, out_dtype=torch.float16)
    assert (got16.float() - ref.half().float()).abs().max() <= 2.0 ** -24 + ref.abs().max() * 2.0 ** -10


def test_int8_weight_quantizer_round_trip():
    """quantize (rotate, rowmax/127, round; tests/test_fp16_safe.py:171-174) then dequantize_rows
    recovers the weight within half a step."""
    w = torch.randn(12, 512, generator=torch.Generator().manual_seed(12))
    q, s = oracle.quantize_weight_int8(w, True, 256)
    back = oracle.dequantize_rows(q, s, True, 256, torch.float32)
    # rotation is orthonormal: the error norm per row is at most sqrt(K) * s/2
    err = (back - w).norm(dim=1)
    assert torch.all(err <= (512 ** 0.5) * s.squeeze(1) * 0.5 * 1.001)


# ------------------------------------------------------------------ fp8 quantize
def _e4m3_values():
    """Every finite OCP e4m3fn value (torch's decode of all 256 codes)."""
    vals = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    return vals[torch.isfinite(vals)]


def test_quantize_fp8_known_rows_without_rotation():
    """x = v * 2^-e with v e4m3-representable and max|v| = 448 -> codes are v's codes (torch's
    cast) and the scale is 2^-e exactly: r = 448 / amax = 2^e, so u r = v is exact."""
    g = torch.Generator().manual_seed(31)
    vals = _e4m3_values()
    v = vals[torch.randint(0, vals.numel(), (16, 256), generator=g)]
    v[:, 11] = 448.0
    v[::2, 11] = -448.0
    e = torch.arange(16) - 8
    x64 = v.double() * torch.pow(2.0, -e.double())[:, None]
    x = x64.to(torch.bfloat16)
    assert torch.equal(x.double(), x64)           # 4 significant bits: exact in bf16
    q, s = oracle.quantize_rows_fp8(x)
    assert torch.equal(q, v.to(torch.float8_e4m3fn).view(torch.uint8))
    assert torch.equal(s.double(), torch.pow(2.0, -e.double()))


def test_quantize_fp8_ties_round_to_even():
    """scale 1 (absmax 448): midpoints go to the even mantissa, in the normal and subnormal range."""
    x = torch.tensor([[448.0, 1.0625, 1.1875, -1.0625, -1.1875, 2.0 ** -10, 3 * 2.0 ** -10, 13.0,
                       15.0, -0.0] + [0.0] * 6], dtype=torch.bfloat16)
    q, s = oracle.quantize_rows_fp8(x)
    assert s.item() == 1.0
    got = q[0, :10].view(torch.float8_e4m3fn).float().tolist()
    # 1.0625 between 1 (m=0) and 1.125 (m=1) -> 1; 1.1875 between 1.125 (m=1) and 1.25 (m=2) -> 1.25;
    # 2^-10 between 0 and 2^-9 -> 0; 3 2^-10 between 2^-9 (m=1) and 2^-8 (m=2) -> 2^-8;
    # 13 between 12 (m=4) and 14 (m=6)... representable (m=5 at [8,16) has step 1): 13 stays;
    # 15 is 15 (m=7)
    assert got == [448.0, 1.0, 1.25, -1.0, -1.25, 0.0, 2.0 ** -8, 13.0, 15.0, -0.0]


def test_quantize_fp8_static_scale_saturates():
    x = torch.tensor([[1000.0, -1000.0, 0.25, 0.0] + [0.0] * 12], dtype=torch.bfloat16)
    q, s = oracle.quantize_rows_fp8(x, static_scale=0.5)
    assert s.item() == 0.5
    assert q[0, :4].view(torch.float8_e4m3fn).float().tolist() == [448.0, -448.0, 0.5, 0.0]


def test_quantize_fp8_zero_row():
    x = torch.zeros(3, 64, dtype=torch.bfloat16)
    x[1, 5] = 2.0
    q, s = oracle.quantize_rows_fp8(x)
    assert s[0].item() == 1.0 and s[2].item() == 1.0 and int(q[0].sum()) == 0 and int(q[2].sum()) == 0
    assert s[1].item() == np.float32(np.float32(2.0) / np.float32(448.0)) and q[1, 5].view(torch.float8_e4m3fn).item() == 448.0


@pytest.mark.parametrize("g", [0, 16, 256])
def test_quantize_fp8_matches_torch_restatement(g):
    """Per-row absmax (torch amax), r = 448 / a in fp32, clamp, torch's own e4m3fn cast: equal to
    the oracle's C loop and codec.  The rotated case takes the normalized rotation (pinned above):
    scaling by 2^-k commutes with the division and the product, so u r and the scale are unchanged."""
    x = heavy_rows_cpu(24, 2048, seed=40 + g)
    u = oracle.rotate_rows(x, g) if g else x.float()
    a = u.abs().amax(1, keepdim=True)
    r = torch.tensor(448.0) / a
    codes = (u * r).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
    scale = (a / torch.tensor(448.0)).reshape(-1)
    q, s = oracle.quantize_rows_fp8(x, g)
    assert torch.equal(q, codes)
    assert torch.equal(s, scale)
    # planted mistake: a per-tensor instead of per-row scale is caught
    wrong = (u * (448.0 / u.abs().max())).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
    assert not torch.equal(q, wrong)


@pytest.mark.parametrize("fp8", [False, True])
def test_quantize_nan_row_convention(fp8):
    """A NaN in a row makes its scale NaN (torch's amax propagates NaN), so the row's dequantized
    output is NaN; its codes are the lower bound (fmax(NaN, -LIM)); other rows are untouched."""
    x = heavy_rows_cpu(4, 512, seed=5)
    x[2, 100] = float("nan")
    fn = oracle.quantize_rows_fp8 if fp8 else oracle.quantize_rows_i8
    for g in (0, 256):
        q, s = fn(x, g)
        assert torch.isnan(s[2]) and not torch.isnan(s[[0, 1, 3]]).any()
        assert torch.isnan(x.float()[2].abs().amax())            # torch's convention
        low = torch.full((512,), 0xFE, dtype=torch.uint8) if fp8 else torch.full((512,), -127, dtype=torch.int8)
        assert torch.equal(q[2], low)
        clean = x.clone()
        clean[2] = 0
        qc, sc = fn(clean, g)
        assert torch.equal(q[[0, 1, 3]], qc[[0, 1, 3]]) and torch.equal(s[[0, 1, 3]], sc[[0, 1, 3]])


# -------------------------------------------------------------------- fp8 decode
@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_dequant_fp8_matches_torch_decode(per_row, out_dtype):
    """round_out(e4m3(q) * s): torch's float8_e4m3fn decode times the fp32 scale, then torch's cast."""
    g = torch.Generator().manual_seed(41)
    codes = torch.randint(0, 256, (37, 96), generator=g, dtype=torch.uint8)
    codes[codes == 0x7F] = 0x7E
    codes[codes == 0xFF] = 0xFE
    s = torch.rand(37, generator=g) * 1e-2 + 1e-4 if per_row else torch.tensor(3.1e-3)
    got = oracle.dequant_fp8(codes, s, out_dtype)
    ref = (codes.view(torch.float8_e4m3fn).float() * (s[:, None] if per_row else s)).to(out_dtype)
    assert torch.equal(got.view(torch.int16) if out_dtype != torch.float32 else got,
                       ref.view(torch.int16) if out_dtype != torch.float32 else ref)


def heavy_rows_cpu(M, K, seed):
    """N(0,1) rows with 1% of channels x20, bf16 (the activation recipe of the GPU tests)."""
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=gen)
    idx = torch.randperm(K, generator=gen)[: max(1, K // 100)]
    x[:, idx] *= 20
    return x.to(torch.bfloat16)
