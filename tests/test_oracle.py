"""Pins the CPU oracle against what mathematics and library routines fix (no GPU)."""

import math
import numpy as np
import pytest
import torch

from oracle import nf4_oracle as o


# ------------------------------------------------------------------------------- NF4 table

def test_nf4_table_matches_closed_form():
    built = o.create_normal_map()
    assert built.shape == (16,)
    np.testing.assert_allclose(built, o.NF4_CODE, rtol=0, atol=1e-6)


def test_nf4_table_invariants():
    c = o.NF4_CODE
    assert c.dtype == np.float32 and c.shape == (16,)
    assert np.all(np.diff(c) > 0)
    assert c[0] == -1.0 and c[15] == 1.0 and c[7] == 0.0
    assert (c > 0).sum() == 8 and (c < 0).sum() == 7
    # literals are exact fp32 values
    assert np.all(c.astype(np.float64).astype(np.float32) == c)


# ----------------------------------------------------------------------------- dynamic map

def test_dynamic_map_closed_form():
    d = o.DYNAMIC_CODE.astype(np.float64)
    assert d.shape == (256,) and np.all(np.diff(d) > 0)
    assert d[0] < 0 and d[-1] == 1.0 and (d == 0).sum() == 1
    pos = d[(d > 0) & (d < 1.0)]
    neg = -d[d < 0][::-1]
    np.testing.assert_array_equal(np.sort(pos), np.sort(neg))
    expected = []
    for i in range(7):
        b = np.linspace(0.1, 1.0, 2 ** i + 1)
        expected += list(10.0 ** (i - 6) * (b[:-1] + b[1:]) / 2)
    np.testing.assert_allclose(np.sort(pos), np.sort(expected), rtol=1e-6)
    # per decade: 2**i values in (10**(i-6) * 0.1, 10**(i-6)]
    for i in range(7):
        lo, hi = 10.0 ** (i - 6) * 0.1, 10.0 ** (i - 6)
        assert ((pos > lo) & (pos <= hi)).sum() == 2 ** i


# -------------------------------------------------------------------------------- dequant

def _small(shape=(24, 128), seed=0, scale=0.02, bs=64, nested=True):
    w = np.random.default_rng(seed).standard_normal(shape).astype(np.float32) * scale
    return w, *o.quantize_nf4(w, blocksize=bs, compress_statistics=nested)


@pytest.mark.parametrize("nested", [True, False])
@pytest.mark.parametrize("shape,bs", [((24, 128), 64), ((5, 7), 64), ((3, 33), 2), ((17, 256), 128)])
def test_dequant_vectorised_equals_element_loop(shape, bs, nested):
    _, packed, st = _small(shape, bs=bs, nested=nested)
    np.testing.assert_array_equal(o.dequantize(packed, st, "f16"), o.dequantize_loop(packed, st))


def test_absmax_rebuild_matches_scalar_loop():
    _, packed, st = _small((40, 512))
    a = o.absmax_fp32(st)
    for b in range(st.absmax.size):
        prod = np.float32(st.state2.code[st.absmax[b]]) * np.float32(st.state2.absmax[b // 256])
        assert a[b] == np.float32(np.float32(prod) + np.float32(st.offset))


def test_absmax_rebuild_has_no_fma():
    # a case where fma(x, y, z) and fp32(fp32(x*y) + z) differ: the oracle must give the latter
    x, y, z = np.float32(1.0 + 2 ** -12), np.float32(1.0 + 2 ** -12), np.float32(-1.0)
    prod = np.float32(x * y)
    separate = np.float32(prod + z)
    fused = np.float32(np.float64(x) * np.float64(y) + np.float64(z))
    assert separate != fused
    st = o.OracleQuantState(absmax=np.array([1], np.uint8), shape=(1, 64), nested=True,
                            offset=float(z),
                            state2=o.OracleState2(absmax=np.array([y], np.float32),
                                                  code=np.array([0.0, x] + [0.0] * 254,
                                                                np.float32)))
    assert o.absmax_fp32(st)[0] == separate


def test_dequant_conversions_match_torch():
    _, packed, st = _small((64, 256))
    f32 = o.dequantize_f32(packed, st)
    t = torch.from_numpy(f32)
    np.testing.assert_array_equal(o.dequantize(packed, st, "f16"), t.half().numpy())
    bf = torch.from_numpy(o.dequantize(packed, st, "bf16").view(np.int16)).view(torch.bfloat16)
    assert torch.equal(bf, t.bfloat16())


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("nested", [True, False])
def test_scaled_codes_match_torch_and_element_loop(dtype, nested):
    """The decode GEMV's weight value round(fp32(round(code[nib])) * absmax) restated three ways:
    the vectorised oracle, torch's own conversions, and an element loop; where the code is
    exact in the dtype (+-1, 0) it equals the dequantized weight."""
    _, packed, st = _small((16, 256), nested=nested)
    got = o.dequantize_scaled_codes(packed, st, dtype).reshape(-1)
    tdt = torch.float16 if dtype == "f16" else torch.bfloat16
    code = torch.from_numpy(st.code.astype(np.float32)).to(tdt).float()
    nib = torch.from_numpy(o.nibbles(packed, 16 * 256).astype(np.int64))
    a = torch.from_numpy(o.absmax_fp32(st))[torch.arange(16 * 256) // st.blocksize]
    ref = (code[nib] * a).to(tdt)
    got_t = torch.from_numpy(got.view(np.int16)).view(tdt) if dtype == "bf16" else \
        torch.from_numpy(got)
    assert torch.equal(got_t, ref)
    p = packed.reshape(-1)
    ab = o.absmax_fp32(st)
    for i in range(0, 16 * 256, 97):
        nb = (int(p[i // 2]) >> 4) if i % 2 == 0 else (int(p[i // 2]) & 0xF)
        c = np.float32(torch.tensor(float(st.code[nb])).to(tdt).float().item())
        v = np.float32(c * ab[i // st.blocksize])
        assert torch.equal(torch.tensor(v).to(tdt), ref[i:i + 1].reshape(()))
    exact = np.isin(nib.numpy(), [0, 7, 15])
    plain = o.dequantize(packed, st, dtype).reshape(-1)
    np.testing.assert_array_equal(got[exact].view(np.int16), plain[exact].view(np.int16))


def test_bf16_rounding_ties_to_even():
    vals = np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -(1.0 + 2 ** -8), 1.0 + 2 ** -9,
                     3.0e38, 1e-40], np.float32)
    ours = torch.from_numpy(o.f32_to_bf16_bits(vals).view(np.int16)).view(torch.bfloat16)
    assert torch.equal(ours, torch.from_numpy(vals).bfloat16())


def test_dequant_special_cases():
    # absmax exactly 1.0 (no double quant): every element is its code value rounded to fp16
    n = 64
    q = np.arange(n, dtype=np.uint8) % 16
    packed = ((q[0::2] << 4) | q[1::2]).astype(np.uint8)
    st = o.OracleQuantState(absmax=np.ones(1, np.float32), shape=(1, n))
    out = o.dequantize(packed, st, "f16").reshape(-1)
    np.testing.assert_array_equal(out, o.NF4_CODE[q].astype(np.float16))
    # code 7 is zero whatever the absmax; code 15 gives the absmax itself
    st.absmax = np.array([3.5], np.float32)
    out = o.dequantize(packed, st, "f16").reshape(-1)
    assert np.all(out[q == 7] == 0) and np.all(out[q == 15] == np.float16(3.5))
    assert np.all(out[q == 0] == np.float16(-3.5))
    # high nibble first: byte 0xF0 -> [code15, code0]
    st = o.OracleQuantState(absmax=np.ones(1, np.float32), shape=(1, 2))
    np.testing.assert_array_equal(o.dequantize(np.array([0xF0], np.uint8), st, "f16").reshape(-1),
                                  np.array([1.0, -1.0], np.float16))


def test_quantize_roundtrip_error_bound():
    w, packed, st = _small((64, 512), seed=3)
    deq = o.dequantize_f32(packed, st).reshape(-1)
    a = o.absmax_fp32(st)
    true_absmax = np.abs(w.reshape(-1, 64)).max(1)
    # per block: |w - deq| <= |a| * half the widest NF4 gap + |a - true absmax|
    err = np.abs(w.reshape(-1) - deq).reshape(-1, 64).max(1)
    bound = np.abs(a) * o.nf4_max_gap() + np.abs(a - true_absmax) + 1e-7
    assert np.all(err <= bound)
    # the double-quantized absmax is close to the true one (8-bit dynamic code)
    assert np.max(np.abs(a - true_absmax) / true_absmax) < 0.02


def test_quantize_zero_block():
    w = np.zeros((2, 64), np.float32)
    w[1] = np.linspace(-1, 1, 64, dtype=np.float32)
    packed, st = o.quantize_nf4(w)
    deq = o.dequantize_f32(packed, st)
    assert np.all(o.nibbles(packed, 128)[:64] == 7)
    assert np.all(np.isfinite(deq))


def test_quantize_nearest_code():
    x = np.array([-1.0, -0.9, 0.0, 0.03, 0.05, 0.99, 1.0], np.float32)
    got = o.quantize_nf4_codes(x)
    brute = np.array([np.argmin(np.abs(o.NF4_CODE.astype(np.float64) - v)) for v in x])
    np.testing.assert_array_equal(got, brute)


# ------------------------------------------------------------------------ GEMM / LoRA refs

def test_lora_backward_formulas_match_autograd():
    g = torch.Generator().manual_seed(0)
    m, k, n, r, s = 9, 32, 24, 4, 2.0
    x = torch.randn(m, k, generator=g, requires_grad=True)
    w = torch.randn(n, k, generator=g)
    a = torch.randn(r, k, generator=g, requires_grad=True)
    b = torch.randn(8, r, generator=g, requires_grad=True)
    lor = [(4, 8, x, a, b, s)]
    y = x @ w.t()
    y = torch.cat([y[:, :4], y[:, 4:12] + s * (x @ a.t()) @ b.t(), y[:, 12:]], 1)
    dy = torch.randn(m, n, generator=g)
    y.backward(dy)
    ref_fwd = o.linear_fwd(x.detach(), w, None, [(4, 8, x.detach(), a.detach(), b.detach(), s)])
    torch.testing.assert_close(ref_fwd, y.detach())
    dx = o.linear_dx(dy, w, [(4, 8, None, a.detach(), b.detach(), s)])
    torch.testing.assert_close(dx, x.grad)
    ga, gb = o.lora_grads(dy[:, 4:12], x.detach(), a.detach(), b.detach(), s)
    torch.testing.assert_close(ga, a.grad)
    torch.testing.assert_close(gb, b.grad)
    assert lor


def test_mlp_reference_matches_autograd_composition():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(5, 16, generator=g)
    wg, wu, wd = (torch.randn(32, 16, generator=g), torch.randn(32, 16, generator=g),
                  torch.randn(16, 32, generator=g))
    ref = torch.nn.functional.linear(
        torch.nn.functional.silu(x @ wg.t()) * (x @ wu.t()), wd)
    torch.testing.assert_close(o.mlp_fwd(x, wg, wu, wd), ref)


def test_rel_errors_definition():
    ref = torch.tensor([1.0, -2.0, 4.0])
    out = torch.tensor([1.0, -2.0, 4.4])
    mx, mean = o.rel_errors(out, ref)
    assert abs(mx - 0.1) < 1e-6 and abs(mean - (0.4 / 3) / (7 / 3)) < 1e-6


# ------------------------------------------------------------ norm and RoPE restatements

def _norm_inputs(rows=5, cols=24, seed=0):
    import torch

    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g)  # noqa: E731
    keep = lambda: (torch.rand(rows, cols, generator=g) > 0.3).float()  # noqa: E731
    return r(rows, cols), r(rows, cols) * 0.5, r(cols).abs() + 0.5, keep(), keep()


def test_keep_bits_known_answer_and_numpy():
    """The mask packing (layer.py:76-90): bit k of byte j is element 8 j + k, q's bytes before
    v's in a row.  Pinned by hand-worked bytes and by numpy's little-endian packbits; the
    unpacking inverts it."""
    kq = np.zeros((2, 16), np.uint8)
    kv = np.zeros((2, 16), np.uint8)
    kq[0, 0] = 1            # element 0 -> byte 0 bit 0
    kq[0, 9] = 1            # element 9 -> byte 1 bit 1
    kv[0, 7] = 1            # v element 7 -> v byte 0 bit 7
    kv[1, 8:16] = 1         # v byte 1 all set
    p = o.pack_keep_bits(kq, kv)
    assert p.shape == (2, 4) and p.dtype == np.uint8
    assert p[0].tolist() == [0x01, 0x02, 0x80, 0x00]
    assert p[1].tolist() == [0x00, 0x00, 0x00, 0xFF]
    rng = np.random.default_rng(7)
    kq = (rng.random((5, 96)) > 0.1).astype(np.uint8)
    kv = (rng.random((5, 96)) > 0.5).astype(np.uint8)
    p = o.pack_keep_bits(kq, kv)
    np.testing.assert_array_equal(p[:, :12], np.packbits(kq, axis=1, bitorder="little"))
    np.testing.assert_array_equal(p[:, 12:], np.packbits(kv, axis=1, bitorder="little"))
    uq, uv = o.unpack_keep_bits(p, 96)
    np.testing.assert_array_equal(uq, kq)
    np.testing.assert_array_equal(uv, kv)


def test_add_rmsnorm_matches_row_loop():
    """The vectorised norm against an explicit per-row, per-element fp64 loop."""
    x, d, w, kq, kv = _norm_inputs()
    y, rstd, oq, ov = o.add_rmsnorm(x, w, 1e-6, d=d, keep_q=kq, keep_v=kv, scale_q=1.25, scale_v=0.5)
    for r in range(x.shape[0]):
        h = [float(x[r, c]) + float(d[r, c]) for c in range(x.shape[1])]
        rs = 1.0 / math.sqrt(sum(v * v for v in h) / len(h) + 1e-6)
        assert abs(float(rstd[r]) - rs) <= 1e-6 * rs
        for c in range(x.shape[1]):
            yy = float(w[c]) * h[c] * rs
            assert abs(float(y[r, c]) - yy) <= 1e-5 * (1 + abs(yy))
            assert abs(float(oq[r, c]) - yy * float(kq[r, c]) * 1.25) <= 1e-5 * (1 + abs(yy))
            assert abs(float(ov[r, c]) - yy * float(kv[r, c]) * 0.5) <= 1e-5 * (1 + abs(yy))


def test_rmsnorm_bwd_matches_autograd():
    """The hand-written norm gradient (output, both dropout branches, residual) against torch
    autograd of the forward restatement."""
    import torch

    x, d, w, kq, kv = _norm_inputs(seed=1)
    g = torch.Generator().manual_seed(2)
    gy, gq, gv, gres = (torch.randn(x.shape, generator=g) for _ in range(4))
    xa, da = x.clone().requires_grad_(), d.clone().requires_grad_()
    y, rstd, oq, ov = o.add_rmsnorm(xa, w, 1e-6, d=da, keep_q=kq, keep_v=kv, scale_q=2.0, scale_v=3.0)
    ((y * gy).sum() + (oq * gq).sum() + (ov * gv).sum()).backward()
    dx = o.rmsnorm_bwd(x, w, rstd.detach(), dy=gy, d=d, dres=gres, dq=gq, dv=gv, keep_q=kq,
                       keep_v=kv, scale_q=2.0, scale_v=3.0)
    torch.testing.assert_close(dx, xa.grad + gres, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(da.grad, xa.grad)  # x and d enter as one sum


def _rope_inputs(tokens=3, n_heads=6, n_kv=2, head_dim=8, seed=3):
    import torch

    g = torch.Generator().manual_seed(seed)
    qkv = torch.randn(tokens, (n_heads + 2 * n_kv) * head_dim, generator=g)
    ang = torch.rand(tokens, head_dim // 2, generator=g) * 6.0
    cos = torch.cat([ang.cos(), ang.cos()], 1)
    sin = torch.cat([ang.sin(), ang.sin()], 1)
    return qkv, cos, sin


def test_qkv_rope_identity_norms_and_expansion():
    """cos = 1, sin = 0 is the identity; a rotation keeps every pair's norm; k and v copies of
    one group are identical and equal the caches."""
    import torch

    qkv, cos, sin = _rope_inputs()
    nh, nkv, hd = 6, 2, 8
    q, k, v, kc, vc = o.qkv_rope(qkv, torch.ones_like(cos), torch.zeros_like(sin), nh, nkv, hd)
    assert torch.equal(q.reshape(3, -1), qkv[:, :nh * hd])
    q, k, v, kc, vc = o.qkv_rope(qkv, cos, sin, nh, nkv, hd)
    qin = qkv[:, :nh * hd].reshape(3, nh, hd)
    pair = lambda t: t[..., :hd // 2] ** 2 + t[..., hd // 2:] ** 2  # noqa: E731
    torch.testing.assert_close(pair(q), pair(qin))
    for h in range(nh):
        assert torch.equal(k[:, h], kc[:, h // 3]) and torch.equal(v[:, h], vc[:, h // 3])
    assert torch.equal(vc.reshape(3, -1), qkv[:, (nh + nkv) * hd:])


def test_qkv_rope_sign_known_answer():
    """The rotation's sign convention (layer.py:196-197, the rotate-half form of Qwen2's
    apply_rotary_pos_emb): at cos = 0, sin = 1 every pair (lo, hi) becomes (-hi, lo); at
    cos = 0, sin = -1 it becomes (hi, -lo).  An exchanged or flipped sign fails one of the two."""
    import torch

    qkv, cos, sin = _rope_inputs(seed=7)
    nh, nkv, hd = 6, 2, 8
    half = hd // 2
    for s in (1.0, -1.0):
        q, k, _, kc, _ = o.qkv_rope(qkv, torch.zeros_like(cos), torch.full_like(sin, s), nh, nkv, hd)
        qin = qkv[:, :nh * hd].reshape(3, nh, hd)
        kin = qkv[:, nh * hd:(nh + nkv) * hd].reshape(3, nkv, hd)
        for got, src in ((q, qin), (kc, kin)):
            assert torch.equal(got[..., :half], -s * src[..., half:])
            assert torch.equal(got[..., half:], s * src[..., :half])


def test_qkv_rope_bwd_matches_autograd():
    import torch

    qkv, cos, sin = _rope_inputs(seed=4)
    g = torch.Generator().manual_seed(5)
    gq, gk, gv = (torch.randn(3, 6, 8, generator=g) for _ in range(3))
    qa = qkv.clone().requires_grad_()
    q, k, v, _, _ = o.qkv_rope(qa, cos, sin, 6, 2, 8)
    ((q * gq).sum() + (k * gk).sum() + (v * gv).sum()).backward()
    torch.testing.assert_close(o.qkv_rope_bwd(gq, gk, gv, cos, sin, 2), qa.grad)


# ------------------------------------------------------------------ int8 input gradients

def test_round_i8_known_answers():
    """Ties away from zero and the clamp (layer.py:299-303), evaluated in fp32: v + 0.5 rounds
    in fp32 before the floor, so the largest float below 0.5 goes to 1 as it does there."""
    v = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 0.49, -0.49, 126.5, 127.6, -300.0, 0.0,
                  np.nextafter(np.float32(0.5), np.float32(0))], dtype=np.float32)
    assert o.round_i8(v).tolist() == [1, 2, 3, -1, -2, -3, 0, 0, 127, 127, -127, 0, 1]


def _i8_weights(seed, shapes, nested=True):
    g = np.random.default_rng(seed)
    return [o.quantize_nf4(g.standard_normal((r, c)).astype(np.float32) * 0.02,
                           compress_statistics=nested) for r, c in shapes]


def test_int8_rows_invariants():
    """Each row's largest |x| maps to +-127, every value lies within half a step of q * s, and
    s = largest / 127."""
    g = np.random.default_rng(7)
    x = (g.standard_normal((20, 96)) * np.logspace(-3, 2, 20)[:, None]).astype(np.float32)
    q, s = o.int8_rows(x)
    top = np.abs(x).max(axis=1)
    assert np.array_equal(s, (top / np.float32(127)).astype(np.float32))
    assert np.array_equal(np.abs(q[np.arange(20), np.abs(x).argmax(axis=1)]), np.full(20, 127))
    assert np.all(np.abs(q.astype(np.float64) * s[:, None] - x) <= 0.5 * s[:, None] * (1 + 1e-5))
    q0, s0 = o.int8_rows(np.zeros((2, 8), np.float32))  # empty rows: scale 1e-20 / 127
    assert not q0.any() and np.all(s0 > 0)


def test_int8_matmul_is_exact():
    g = np.random.default_rng(8)
    a = g.integers(-127, 128, (5, 7), dtype=np.int8)
    b = g.integers(-127, 128, (3, 7), dtype=np.int8)
    ref = [[sum(int(a[i, k]) * int(b[j, k]) for k in range(7)) for j in range(3)] for i in range(5)]
    assert o.int8_matmul(a, b).tolist() == ref
    big = np.full((1, 17920), 127, np.int8)
    assert int(o.int8_matmul(big, big)[0, 0]) == 127 * 127 * 17920  # fits int32


def test_int8_col_scales_and_weights():
    """Column scales from the dtype-rounded weights (torch's amax over the fp16 / bf16
    dequantized stack, an independent route), and the transposed int8 stack within half a
    step of the fp32 weights (the reference test's 0.6 scale bound, test_kernels.py:344-346)."""
    ws = _i8_weights(9, [(128, 192), (64, 192)])
    for dt in ("f16", "bf16"):
        w = torch.cat([torch.from_numpy(o.dequantize(p, st, dt).view(np.int16)).view(
            torch.bfloat16 if dt == "bf16" else torch.float16).float() for p, st in ws])
        ref = (w.abs().amax(0).clamp_min(1e-20) / 127).numpy()
        assert np.array_equal(o.col_scales(ws, dt), ref.astype(np.float32))
    cs = o.col_scales(ws)
    qt = o.int8_weight_t(ws, cs)
    wf = o.stack_f32(ws)
    assert qt.shape == (192, 192) and qt.dtype == np.int8
    assert np.all(np.abs(qt.T.astype(np.float64) * cs[None, :] - wf) <= 0.5 * cs[None, :] * 1.01)
    q, s = o.int8_weight_rows(ws)
    assert np.all(np.abs(q.astype(np.float64) * s[:, None] - wf) <= 0.5 * s[:, None] * 1.01)


def test_int8_swiglu_bwd_against_float64():
    """The SwiGLU gradients before requantization agree with a float64 evaluation of the same
    formula, and the int8 codes reproduce them within half a step."""
    g = np.random.default_rng(10)
    m, inter = 6, 40
    acc = g.integers(-40000, 40000, (m, inter)).astype(np.int64)
    sd = (g.random(m) * 1e-3 + 1e-4).astype(np.float32)
    cs = (g.random(inter) * 1e-3 + 1e-4).astype(np.float32)
    gu = (g.standard_normal((m, 2 * inter)) * 2).astype(np.float16).astype(np.float32)
    q, sq, dg, du = o.int8_swiglu_bwd(acc, sd, cs, gu)
    d = acc.astype(np.float64) * sd[:, None] * cs[None, :]
    gg, uu = gu[:, :inter].astype(np.float64), gu[:, inter:].astype(np.float64)
    sig = 1 / (1 + np.exp(-gg))
    np.testing.assert_allclose(dg, d * uu * sig * (1 + gg * (1 - sig)), rtol=2e-5, atol=1e-12)
    np.testing.assert_allclose(du, d * gg * sig, rtol=2e-5, atol=1e-12)
    both = np.concatenate([dg, du], axis=1)
    assert np.all(np.abs(q.astype(np.float64) * sq[:, None] - both) <= 0.5 * sq[:, None] * 1.01)
    assert np.array_equal(np.abs(q).max(axis=1), np.full(m, 127))


def test_int8_mlp_dx_against_fp32():
    """The composite int8 MLP input gradient against the fp32 one on the same dequantized
    weights: within 3e-2 of the largest |dy2| (two int8 products, each held to 2e-2 by the
    reference's own test, test_kernels.py:350, 357)."""
    g = np.random.default_rng(11)
    n, hidden, inter = 96, 256, 384
    gate, up = _i8_weights(12, [(inter, hidden), (inter, hidden)])
    down = _i8_weights(13, [(hidden, inter)])[0]
    x = torch.from_numpy(g.standard_normal((n, hidden)).astype(np.float32)).half()
    wg, wu, wd = (torch.from_numpy(o.dequantize(p, st)).float() for p, st in (gate, up, down))
    gu = torch.cat([x.float() @ wg.t(), x.float() @ wu.t()], 1).half()
    dh2 = torch.from_numpy(g.standard_normal((n, hidden)).astype(np.float32) * 1e-2)
    dy2 = o.mlp_dx_int8(dh2, gu, [gate, up], [down])
    gg, uu = gu.float()[:, :inter], gu.float()[:, inter:]
    sig = torch.sigmoid(gg)
    dact = dh2 @ wd
    ref = torch.cat([dact * uu * sig * (1 + gg * (1 - sig)), dact * gg * sig], 1) @ torch.cat([wg, wu])
    err = np.abs(dy2 - ref.numpy()).max() / np.abs(ref.numpy()).max()
    assert err <= 3e-2, err


def test_int8_gate_up_fwd_against_fp32():
    """The int8 gate|up forward: gate|up within 2e-2 of the largest fp32 product (the
    reference's own bound for one int8 product, test_kernels.py:350) and on the dtype's grid;
    act against torch's fp32 SiLU (torch.nn.functional.silu, a library routine) times up on the
    rounded halves, within one rounding to the dtype.  A swapped gate / up, a scale taken per
    column instead of per row, or a missing rounding of the halves fails one of these."""
    ws = _i8_weights(14, [(256, 192), (256, 192)])
    g = np.random.default_rng(15)
    x = torch.from_numpy((g.standard_normal((40, 192)) * np.logspace(-2, 1, 40)[:, None])
                         .astype(np.float32)).half()
    w = torch.from_numpy(o.stack_f32(ws))
    ref = x.float() @ w.t()
    for dt, ulp, tiny in (("f16", 2.0 ** -10, 2.0 ** -24), ("bf16", 2.0 ** -7, 1e-38)):
        gu, act = o.gate_up_fwd_int8(x.float().numpy(), ws, dt)
        assert gu.shape == (40, 512) and act.shape == (40, 256)
        err = np.abs(gu - ref.numpy()).max(axis=1) / np.abs(ref.numpy()).max(axis=1)
        assert err.max() <= 2e-2, err.max()
        assert np.array_equal(o._round_to(gu, dt), gu)
        gg, uu = torch.from_numpy(gu[:, :256]), torch.from_numpy(gu[:, 256:])
        want = (torch.nn.functional.silu(gg) * uu).numpy()
        assert np.all(np.abs(act - want) <= np.abs(want) * ulp + tiny)  # tiny: fp16 subnormals
        assert np.array_equal(o._round_to(act, dt), act)
