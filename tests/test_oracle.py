"""Pins the CPU oracle before it is trusted as the checker of the HIP path.

Each check is chosen so that a plausible mistake in the oracle (a dropped
term, a transposed operand, a misplaced scale, a wrong segment index) fails:
brute-force loops, finite differences, torch.autograd on an independent
restatement, the reference's own construction fixture, and invariants.
"""
import itertools
import math

import numpy as np
import pytest
import torch

from oracle import multilora_oracle as O
from oracle import torch_reference as TR


def _case(rng, M=9, K=6, N=5, ranks=(2, 3), lengths=(3, 0, 2, 4), ids=(0, 1, -1, 1), bias=True):
    x = rng.standard_normal((M, K))
    w = rng.standard_normal((N, K))
    b = rng.standard_normal(N) if bias else None
    As = [rng.standard_normal((r, K)) for r in ranks]
    Bs = [rng.standard_normal((N, r)) for r in ranks]
    off = np.concatenate([[0], np.cumsum(lengths)]).astype(int).tolist()
    assert off[-1] == M
    return x, w, b, As, Bs, off, list(ids)


# ---------------------------------------------------------------- bf16 rounding

def test_bf16_round_known_values():
    one = 1.0
    ulp = 2.0 ** -7  # bf16 spacing in [1, 2)
    vals = np.array([one, one + ulp / 2, one + 1.5 * ulp, one + 0.75 * ulp, -one - ulp / 2, 0.0, -0.0,
                     np.inf, -np.inf, 3.0e38], dtype=np.float32)
    want = np.array([one, one, one + 2 * ulp, one + ulp, -one, 0.0, -0.0, np.inf, -np.inf, 2.0 ** 128], dtype=np.float64)
    got = O.bf16_round(vals).astype(np.float64)
    # 3e38 rounds up past the largest bf16 (~3.39e38) only if above; check it stays finite-or-inf consistently
    assert got[:9].tolist() == want[:9].tolist()
    assert np.signbit(got[6])
    assert np.isnan(O.bf16_round(np.array([np.nan], np.float32)))[0]


def test_bf16_round_matches_torch_conversion():
    rng = np.random.default_rng(0)
    v = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 100000),
                        rng.standard_normal(1000).astype(np.float32)]).astype(np.float32)
    want = torch.from_numpy(v).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(O.bf16_round(v), want)


# ---------------------------------------------------------------- forward

def _brute_forward(x, w, b, As, Bs, scales, off, ids):
    M, K = x.shape
    N = w.shape[0]
    y = [[0.0] * N for _ in range(M)]
    for s, a in enumerate(ids):
        for m in range(off[s], off[s + 1]):
            for n in range(N):
                acc = sum(x[m][k] * w[n][k] for k in range(K)) + (b[n] if b is not None else 0.0)
                if a >= 0:
                    r = As[a].shape[0]
                    h = [sum(x[m][k] * As[a][j][k] for k in range(K)) for j in range(r)]
                    acc += scales[a] * sum(h[j] * Bs[a][n][j] for j in range(r))
                y[m][n] = acc
    return np.array(y)


@pytest.mark.parametrize("bias", [True, False])
def test_forward_matches_brute_force(bias):
    rng = np.random.default_rng(1)
    x, w, b, As, Bs, off, ids = _case(rng, bias=bias)
    scales = [0.5, 2.0]
    got = O.forward(x, w, b, As, Bs, scales, off, ids)
    np.testing.assert_allclose(got, _brute_forward(x, w, b, As, Bs, scales, off, ids), rtol=1e-12, atol=1e-12)


def test_forward_rows_and_dx_rows_agree_with_full():
    rng = np.random.default_rng(2)
    x, w, b, As, Bs, off, ids = _case(rng)
    dy = rng.standard_normal((x.shape[0], w.shape[0]))
    rows = [8, 0, 3, 5]
    np.testing.assert_allclose(O.forward_rows(rows, x, w, b, As, Bs, [1.5, 0.25], off, ids),
                               O.forward(x, w, b, As, Bs, [1.5, 0.25], off, ids)[rows], rtol=1e-13)
    dx = O.backward(x, w, As, Bs, [1.5, 0.25], off, ids, dy)[0]
    np.testing.assert_allclose(O.dx_rows(rows, w, As, Bs, [1.5, 0.25], off, ids, dy), dx[rows], rtol=1e-13)


def test_reference_construction_fixture_known_answer():
    """tests/test_training_construction.py:24-38 of the reference: 4x4 Linear filled
    with 0.25, LoRA rank 2 alpha 2 (scale 1), lora_b initialised to zeros -> the
    LoRA linear equals its base: y_n = 0.25 * sum(x) + 0.25."""
    x = np.arange(12, dtype=np.float64).reshape(3, 4) / 7.0
    w = np.full((4, 4), 0.25)
    b = np.full(4, 0.25)
    A = np.random.default_rng(3).uniform(-0.5, 0.5, (2, 4))
    B = np.zeros((4, 2))
    y = O.forward(x, w, b, [A], [B], [2.0 / 2], [0, 3], [0])
    want = np.repeat((0.25 * x.sum(1) + 0.25)[:, None], 4, axis=1)
    np.testing.assert_allclose(y, want, rtol=1e-14)


def test_null_adapter_rows_are_base_only_and_scale_is_linear():
    rng = np.random.default_rng(4)
    x, w, b, As, Bs, off, ids = _case(rng)
    y1 = O.forward(x, w, b, As, Bs, [1.0, 1.0], off, ids)
    y0 = O.forward(x, w, b, As, Bs, [0.0, 0.0], off, ids)
    y3 = O.forward(x, w, b, As, Bs, [3.0, 3.0], off, ids)
    np.testing.assert_allclose(y3 - y0, 3.0 * (y1 - y0), rtol=1e-12, atol=1e-12)
    base = x @ w.T + b
    np.testing.assert_allclose(y0, base, rtol=1e-14)
    lo, hi = off[2], off[3]  # the -1 segment
    np.testing.assert_array_equal(y1[lo:hi], base[lo:hi])


def test_segment_permutation_and_per_role_concatenation():
    rng = np.random.default_rng(5)
    x, w, b, As, Bs, off, ids = _case(rng)
    scales = [0.7, 1.3]
    y = O.forward(x, w, b, As, Bs, scales, off, ids)
    # one call per role (the reference's per-module calls) == the batched call
    for s, a in enumerate(ids):
        lo, hi = off[s], off[s + 1]
        ys = O.forward(x[lo:hi], w, b, As, Bs, scales, [0, hi - lo], [a])
        np.testing.assert_allclose(ys, y[lo:hi], rtol=1e-13)
    # reversing segment order permutes the rows accordingly
    segs = [(off[s], off[s + 1], a) for s, a in enumerate(ids)][::-1]
    order = np.concatenate([np.arange(lo, hi) for lo, hi, _ in segs]).astype(int)
    off2 = np.concatenate([[0], np.cumsum([hi - lo for lo, hi, _ in segs])]).tolist()
    y2 = O.forward(x[order], w, b, As, Bs, scales, off2, [a for _, _, a in segs])
    np.testing.assert_allclose(y2, y[order], rtol=1e-13)


# ---------------------------------------------------------------- backward

def test_backward_matches_finite_differences():
    rng = np.random.default_rng(6)
    x, w, b, As, Bs, off, ids = _case(rng, M=7, K=4, N=3, ranks=(2, 1), lengths=(2, 3, 2, 0), ids=(1, 0, -1, 0))
    scales = [0.9, -1.7]
    dy = rng.standard_normal((7, 3))
    dx, dAs, dBs = O.backward(x, w, As, Bs, scales, off, ids, dy)

    def loss(x_, As_, Bs_):
        return float((O.forward(x_, w, b, As_, Bs_, scales, off, ids) * dy).sum())

    eps = 1e-6

    def numgrad(arr, fn):
        g = np.zeros_like(arr)
        for idx in itertools.product(*map(range, arr.shape)):
            old = arr[idx]
            arr[idx] = old + eps
            fp = fn()
            arr[idx] = old - eps
            fm = fn()
            arr[idx] = old
            g[idx] = (fp - fm) / (2 * eps)
        return g

    np.testing.assert_allclose(dx, numgrad(x, lambda: loss(x, As, Bs)), rtol=1e-6, atol=1e-7)
    for i in range(2):
        np.testing.assert_allclose(dAs[i], numgrad(As[i], lambda: loss(x, As, Bs)), rtol=1e-6, atol=1e-7)
        np.testing.assert_allclose(dBs[i], numgrad(Bs[i], lambda: loss(x, As, Bs)), rtol=1e-6, atol=1e-7)


def test_backward_matches_torch_autograd_of_per_adapter_path():
    rng = np.random.default_rng(7)
    x, w, b, As, Bs, off, ids = _case(rng, M=40, K=16, N=12, ranks=(4, 8), lengths=(10, 12, 8, 10), ids=(1, -1, 0, 1))
    scales = [1.25, 0.5]
    dy = rng.standard_normal((40, 12))
    t = lambda a: torch.from_numpy(np.asarray(a, np.float64))  # noqa: E731
    y, dx, dAs, dBs = TR.per_adapter_step(t(x), t(w), t(b), [t(a) for a in As], [t(v) for v in Bs], scales,
                                          off, ids, t(dy))
    np.testing.assert_allclose(O.forward(x, w, b, As, Bs, scales, off, ids), y.numpy(), rtol=1e-12)
    odx, odAs, odBs = O.backward(x, w, As, Bs, scales, off, ids, dy)
    np.testing.assert_allclose(odx, dx.numpy(), rtol=1e-12)
    for i in range(2):
        np.testing.assert_allclose(odAs[i], dAs[i].numpy(), rtol=1e-12)
        np.testing.assert_allclose(odBs[i], dBs[i].numpy(), rtol=1e-12)


def test_adapter_without_rows_gets_zero_gradient():
    rng = np.random.default_rng(8)
    x, w, b, As, Bs, off, ids = _case(rng, ranks=(2, 3, 2), ids=(0, 1, -1, 1))
    dy = rng.standard_normal((x.shape[0], w.shape[0]))
    _, dAs, dBs = O.backward(x, w, As, Bs, [1, 1, 1], off, ids, dy)
    assert not dAs[2].any() and not dBs[2].any()


# ---------------------------------------------------------------- reference rounding variants

def test_autocast_restatement_matches_torch_cpu_autocast():
    """low_rank.py:28 under bf16 autocast, evaluated by torch's CPU autocast."""
    rng = np.random.default_rng(9)
    M, K, N = 64, 32, 24
    x, w, b, As, Bs, off, ids = _case(rng, M=M, K=K, N=N, ranks=(8, 8), lengths=(30, 34), ids=(0, 1))
    scales = [1.0, 2.0]
    t = lambda a: torch.from_numpy(np.asarray(a, np.float32))  # noqa: E731
    with torch.autocast("cpu", dtype=torch.bfloat16):
        yt = TR.per_adapter_forward(t(x), t(w), t(b), [t(a) for a in As], [t(v) for v in Bs], scales, off, ids)
    assert yt.dtype == torch.bfloat16
    ours = O.forward_autocast_bf16(x, w, b, As, Bs, scales, off, ids)
    # same rounding points; only the fp32 accumulation order inside each product may differ
    assert O.rel_l2(ours, yt.float().numpy()) < 2e-3
    truth = O.forward(O.bf16_round(x), O.bf16_round(w), O.bf16_round(b), [O.bf16_round(a) for a in As],
                      [O.bf16_round(v) for v in Bs], scales, off, ids)
    assert O.rel_l2(ours, truth) < 1e-2


def _torch_variant_inputs(seed):
    rng = np.random.default_rng(seed)
    x, w, b, As, Bs, off, ids = _case(rng, M=64, K=32, N=24, ranks=(8, 8), lengths=(30, 34), ids=(0, 1))
    return x, w, b, As, Bs, off, ids


def test_fp32_update_variant_matches_torch_restatement():
    """native/models.py:44-51: bf16 base module, fp32 update, (base.float() + update*s).to(bf16)."""
    x, w, b, As, Bs, off, ids = _torch_variant_inputs(11)
    scales = [0.5, 2.0]
    xb = torch.from_numpy(np.asarray(x, np.float32)).to(torch.bfloat16)
    wb = torch.from_numpy(np.asarray(w, np.float32)).to(torch.bfloat16)
    bb = torch.from_numpy(np.asarray(b, np.float32)).to(torch.bfloat16)
    outs = []
    for s_, a in enumerate(ids):
        lo, hi = off[s_], off[s_ + 1]
        base = torch.nn.functional.linear(xb[lo:hi], wb, bb)
        A = torch.from_numpy(np.asarray(As[a], np.float32))
        B = torch.from_numpy(np.asarray(Bs[a], np.float32))
        upd = torch.nn.functional.linear(torch.nn.functional.linear(xb[lo:hi].float(), A), B)
        outs.append((base.float() + upd * scales[a]).to(torch.bfloat16))
    want = torch.cat(outs).float().numpy()
    got = O.forward_fp32_update(x, w, b, As, Bs, scales, off, ids)
    assert O.rel_l2(got, want) < 2e-3


def test_livewan_variant_matches_torch_restatement():
    """wanstreamer/lora.py:22-27: y + linear(linear(x.to(fp32), a), b).to(y.dtype) * scale."""
    x, w, b, As, Bs, off, ids = _torch_variant_inputs(12)
    scales = [1.0, 3.0]
    xb = torch.from_numpy(np.asarray(x, np.float32)).to(torch.bfloat16)
    wb = torch.from_numpy(np.asarray(w, np.float32)).to(torch.bfloat16)
    bb = torch.from_numpy(np.asarray(b, np.float32)).to(torch.bfloat16)
    outs = []
    for s_, a in enumerate(ids):
        lo, hi = off[s_], off[s_ + 1]
        y = torch.nn.functional.linear(xb[lo:hi], wb, bb)
        A = torch.from_numpy(np.asarray(As[a], np.float32))
        B = torch.from_numpy(np.asarray(Bs[a], np.float32))
        h = torch.nn.functional.linear(xb[lo:hi].to(torch.float32), A)
        outs.append(y + torch.nn.functional.linear(h, B).to(y.dtype) * scales[a])
    want = torch.cat(outs).float().numpy()
    got = O.forward_livewan(x, w, b, As, Bs, scales, off, ids)
    assert O.rel_l2(got, want) < 2e-3


def test_fp32_update_and_livewan_variants_are_close_to_exact():
    rng = np.random.default_rng(10)
    x, w, b, As, Bs, off, ids = _case(rng, M=64, K=32, N=24, ranks=(8, 8), lengths=(30, 34), ids=(0, 1))
    q = O.bf16_round
    truth = O.forward(q(x), q(w), q(b), As, Bs, [1.0, 1.0], off, ids)
    for fn in (O.forward_fp32_update, O.forward_livewan):
        assert O.rel_l2(fn(x, w, b, As, Bs, [1.0, 1.0], off, ids), truth) < 1e-2


def test_rel_l2_definition():
    assert O.rel_l2([3.0, 4.0], [3.0, 4.0]) == 0.0
    assert math.isclose(O.rel_l2([3.0, 4.0], [0.0, 5.0]), math.hypot(3, 1) / 5.0)


# ------------------------------------------------------------------ e4m3 (quantised base)

def _torch_e4m3_bytes(v):
    return torch.from_numpy(np.asarray(v, np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def _nearest_e4m3(v):
    """Brute force: the finite positive code nearest to |v| (ties to the even code), with v's sign."""
    codes = np.arange(0x7F, dtype=np.uint8)
    vals = O.e4m3_decode(codes).astype(np.float64)
    out = []
    for x in np.asarray(v, np.float64):
        d = np.abs(vals - abs(x))
        best = np.flatnonzero(d == d.min())
        c = int(best[0]) if len(best) == 1 else int(best[(codes[best] & 1) == 0][0])
        out.append(c | (0x80 if math.copysign(1.0, x) < 0 else 0))
    return np.array(out, dtype=np.uint8)


def test_e4m3_decode_matches_torch_for_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    got = O.e4m3_decode(codes)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(got[~np.isnan(got)], want[~np.isnan(want)])
    assert O.e4m3_decode([0x7E])[0] == 448.0 and O.e4m3_decode([0x01])[0] == 2.0 ** -9
    assert O.e4m3_decode([0x08])[0] == 2.0 ** -6 and O.e4m3_decode([0x38])[0] == 1.0


def test_e4m3_encode_matches_torch_and_nearest_value():
    rng = np.random.default_rng(21)
    v = np.concatenate([rng.standard_normal(20000).astype(np.float32) * s for s in (1e-4, 1e-2, 1, 30, 150)])
    v = v[np.abs(v) <= 448]
    pos = O.e4m3_decode(np.arange(0, 0x7F, dtype=np.uint8)).astype(np.float64)
    ties = ((pos[:-1] + pos[1:]) / 2).astype(np.float32)  # exact midpoints, incl. the subnormal grid
    v = np.concatenate([v, ties, -ties, [0.0, -0.0, 448.0, -448.0, 2.0 ** -10, 2.0 ** -6]]).astype(np.float32)
    got = O.e4m3_encode(v)
    assert np.array_equal(got, _torch_e4m3_bytes(v))
    sample = np.concatenate([v[::97], ties])
    assert np.array_equal(O.e4m3_encode(sample), _nearest_e4m3(sample))


def test_e4m3_encode_saturates_past_448():
    v = np.array([448.5, 463.9, 464.0, 500.0, 1e6, -470.0, np.nan], np.float32)
    assert list(O.e4m3_encode(v)) == [0x7E, 0x7E, 0x7E, 0x7E, 0x7E, 0xFE, 0x7E]


def test_quantize_rows_e4m3_properties():
    rng = np.random.default_rng(22)
    x = O.bf16_round(rng.standard_normal((7, 96)) * np.array([1e-3, 1, 1, 50, 1, 1, 1])[:, None])
    x[2] = 0.0
    q, s = O.quantize_rows_e4m3(x)
    assert q.dtype == np.uint8 and s.dtype == np.float32
    assert s[2] == 1.0 and not q[2].any()
    for m in (0, 1, 3, 4, 5, 6):
        amax = np.abs(x[m]).max()
        assert s[m] == np.float32(amax) / np.float32(448)
        assert (q[m] & 0x7F).max() == 0x7E  # the absmax element lands on ±448
        back = O.dequant_rows_e4m3(q[m:m + 1], s[m:m + 1])[0]
        # half an e4m3 ulp: relative 2^-4 in the normal range, absolute 2^-10·s below it
        tol = np.maximum(np.abs(x[m]) * 2.0 ** -4, s[m] * 2.0 ** -10) * (1 + 1e-6)
        assert np.all(np.abs(back - x[m]) <= tol)


def test_fp8_forward_variants_match_brute_force():
    rng = np.random.default_rng(23)
    x, w, b, As, Bs, off, ids = _case(rng, M=9, K=32, N=5, ranks=(2, 3), lengths=(3, 0, 2, 4), ids=(0, 1, -1, 1))
    wq, ws = O.quantize_rows_e4m3(w)
    scales = [0.5, 2.0]
    W = np.array([[float(O.e4m3_decode([wq[n, k]])[0]) * float(ws[n]) for k in range(32)] for n in range(5)])
    xq, xs = O.quantize_rows_e4m3(x)
    Xq = np.array([[float(O.e4m3_decode([xq[m, k]])[0]) * float(xs[m]) for k in range(32)] for m in range(9)])
    aid = O.row_adapters(off, ids)
    want_base, want_q = np.zeros((9, 5)), np.zeros((9, 5))
    for m in range(9):
        for n in range(5):
            lora = 0.0
            if aid[m] >= 0:
                A, B = As[aid[m]], Bs[aid[m]]
                h = [sum(float(x[m, k]) * float(A[j, k]) for k in range(32)) for j in range(A.shape[0])]
                lora = scales[aid[m]] * sum(h[j] * float(B[n, j]) for j in range(A.shape[0]))
            want_base[m, n] = sum(float(x[m, k]) * W[n, k] for k in range(32)) + float(b[n]) + lora
            want_q[m, n] = sum(Xq[m, k] * W[n, k] for k in range(32)) + float(b[n]) + lora
    np.testing.assert_allclose(O.forward_fp8_base(x, wq, ws, b, As, Bs, scales, off, ids), want_base, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(O.forward_fp8_quantized_x(x, wq, ws, b, As, Bs, scales, off, ids), want_q,
                               rtol=1e-12, atol=1e-12)


def test_quantize_rows_e4m3_column_factor():
    """A column factor is one fp32 product before the absmax: with power-of-two
    factors that product is exact, so quantising x·cs equals quantising x with
    the factors; all-ones factors change nothing; the absmax column maps to ±448."""
    rng = np.random.default_rng(24)
    x = O.bf16_round(rng.standard_normal((6, 48)))
    cs = (2.0 ** rng.integers(-6, 7, 48)).astype(np.float32)
    q1, s1 = O.quantize_rows_e4m3(x, col_scale=cs)
    q2, s2 = O.quantize_rows_e4m3((x * cs[None, :]).astype(np.float32))
    assert np.array_equal(q1, q2) and np.array_equal(s1, s2)
    q3, s3 = O.quantize_rows_e4m3(x, col_scale=np.ones(48, np.float32))
    q4, s4 = O.quantize_rows_e4m3(x)
    assert np.array_equal(q3, q4) and np.array_equal(s3, s4)
    cs2 = rng.uniform(0.1, 3.0, 48).astype(np.float32)
    q5, s5 = O.quantize_rows_e4m3(x, col_scale=cs2)
    v = (x * cs2[None, :]).astype(np.float32)
    for m in range(6):
        k = int(np.argmax(np.abs(v[m])))
        assert s5[m] == np.abs(v[m]).max() / np.float32(448) and (q5[m, k] & 0x7F) == 0x7E


def test_fp8_dx_matches_brute_force():
    """dx_fp8_quantized_dy against loops: the base product from the quantised
    dY·w_scale rows, the LoRA term from the exact dY; and, when every dY·w_scale
    row is already on the e4m3 grid at scale 1, equal to the exact dX."""
    rng = np.random.default_rng(25)
    M, K, N = 7, 16, 32
    x, w, b, As, Bs, off, ids = _case(rng, M=M, K=K, N=N, ranks=(2, 3), lengths=(2, 3, 2), ids=(1, -1, 0))
    wq, ws = O.quantize_rows_e4m3(w)  # w [N, K]: W = ws[n]·e4m3(wq[n, k])
    scales = [0.5, 2.0]
    dy = O.bf16_round(rng.standard_normal((M, N)))
    dq, ds = O.quantize_rows_e4m3(dy, col_scale=ws)
    Wd = O.e4m3_decode(wq).astype(np.float64)
    aid = O.row_adapters(off, ids)
    want = np.zeros((M, K))
    for m in range(M):
        for k in range(K):
            base = sum(float(O.e4m3_decode([dq[m, n]])[0]) * Wd[n, k] for n in range(N)) * float(ds[m])
            lora = 0.0
            if aid[m] >= 0:
                A, B = As[aid[m]], Bs[aid[m]]
                g = [sum(float(dy[m, n]) * float(B[n, j]) for n in range(N)) for j in range(A.shape[0])]
                lora = scales[aid[m]] * sum(g[j] * float(A[j, k]) for j in range(A.shape[0]))
            want[m, k] = base + lora
    got = O.dx_fp8_quantized_dy(dy, wq, ws, As, Bs, scales, off, ids)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    # dY·w_scale on the e4m3 grid with row absmax 448: quantisation is exact
    grid = O.e4m3_decode(np.arange(0, 0x7F, dtype=np.uint8))
    dy2 = rng.choice(np.concatenate([grid, -grid]), (M, N)).astype(np.float64)
    dy2[:, 0] = 448.0
    ws1 = np.ones(N, np.float32)
    exact = O.backward(x, Wd, As, Bs, scales, off, ids, dy2)[0]
    np.testing.assert_allclose(O.dx_fp8_quantized_dy(dy2, wq, ws1, As, Bs, scales, off, ids), exact,
                               rtol=1e-12, atol=1e-9)


# ------------------------------------------------------------------ gated residual

def test_gated_residual_rounds_multiply_and_add_separately():
    """bf16(RN(x + RN(y·g))) — helios_residual_kernel.py:66-86. Against torch's float32 ops
    (an independent library doing one rounding per operation), and against a single-rounding
    (fused multiply-add) evaluation, which must differ on some inputs: that pins the order."""
    import torch
    rng = np.random.default_rng(31)
    M, N = 4096, 256
    x = O.bf16_round(rng.standard_normal((M, N)).astype(np.float32))
    y = O.bf16_round(rng.standard_normal((M, N)).astype(np.float32))
    g = rng.standard_normal((4, N)).astype(np.float32)
    got = O.gated_residual(x, y, g, M // 4)
    tx, ty = torch.from_numpy(x), torch.from_numpy(y)
    tg = torch.from_numpy(g).repeat_interleave(M // 4, dim=0)
    want = (tx + ty * tg).to(torch.bfloat16).float().numpy()
    assert np.array_equal(got, want)
    gg = np.repeat(g, M // 4, axis=0).astype(np.float64)
    fused = O.bf16_round((x.astype(np.float64) + y.astype(np.float64) * gg).astype(np.float32))
    assert (fused != got).sum() > 0  # the contraction is observable after bf16 rounding
    # gate rows: row m takes gate row m // gate_rows
    one = O.gated_residual(np.zeros((6, 8), np.float32), np.ones((6, 8), np.float32),
                           np.arange(16, dtype=np.float32).reshape(2, 8), 3)
    assert np.array_equal(one[:3], np.tile(np.arange(8, dtype=np.float32), (3, 1)))
    assert np.array_equal(one[3:], np.tile(np.arange(8, 16, dtype=np.float32), (3, 1)))


def test_gated_residual_f32_is_the_wan_float32_stream():
    """The Wan block's stream (model.py:305-306): x float32, y bf16, e float32, ``x + y * e`` under
    float32 autocast = two float32 roundings and no bf16 rounding. Against torch's float32 ops on
    the same values (an independent evaluation), and against the fused-multiply-add form, which
    must differ on some inputs (the order of the roundings is observable in float32)."""
    import torch
    rng = np.random.default_rng(33)
    M, N = 4096, 256
    x = rng.standard_normal((M, N)).astype(np.float32)
    y = O.bf16_round(rng.standard_normal((M, N)).astype(np.float32))
    g = rng.standard_normal((4, N)).astype(np.float32)
    got = O.gated_residual_f32(x, y, g, M // 4)
    assert got.dtype == np.float32
    tg = torch.from_numpy(g).repeat_interleave(M // 4, dim=0)
    want = (torch.from_numpy(x) + torch.from_numpy(y).to(torch.bfloat16).float() * tg).numpy()
    assert np.array_equal(got, want)
    gg = np.repeat(g, M // 4, axis=0).astype(np.float64)
    fused = (x.astype(np.float64) + y.astype(np.float64) * gg).astype(np.float32)
    assert (fused != got).sum() > 0
    assert (O.bf16_round(got) != got).sum() > 0  # not rounded to bf16
    # the gradient of y through the float32 stream is the same rounded product
    d = rng.standard_normal((64, 32)).astype(np.float32)
    gate = rng.standard_normal((64, 32)).astype(np.float32)
    td = torch.from_numpy(d)
    ty = torch.zeros(64, 32, dtype=torch.bfloat16, requires_grad=True)
    (torch.zeros(64, 32) + ty * torch.from_numpy(gate)).backward(td)
    assert np.array_equal(O.gate_scale(d, gate, 1), ty.grad.float().numpy())


def test_gate_scale_is_one_rounded_product():
    import torch
    rng = np.random.default_rng(32)
    d = O.bf16_round(rng.standard_normal((64, 32)).astype(np.float32))
    g = rng.standard_normal((64, 32)).astype(np.float32)
    got = O.gate_scale(d, g, 1)
    want = (torch.from_numpy(d) * torch.from_numpy(g)).to(torch.bfloat16).float().numpy()
    assert np.array_equal(got, want)


# ------------------------------------------------------------------ modulated LayerNorm

def test_modulated_norm_matches_torch_float32_ops():
    """bf16(RN(RN(v·RN(1 + s)) + h)) against torch's float32 CPU ops, one rounding per
    operation, in the reference's order (wan13b_modulated_norm_kernel.py:70-97); the
    materialization form adds the table rows first (:158-174)."""
    rng = np.random.default_rng(41)
    B, T, W = 2, 64, 96
    v = rng.standard_normal((B, T, W)).astype(np.float32)
    s = (0.1 * rng.standard_normal((B, T, W))).astype(np.float32)
    h = (0.1 * rng.standard_normal((B, T, W))).astype(np.float32)
    tv, ts, th = torch.from_numpy(v), torch.from_numpy(s), torch.from_numpy(h)
    want = (tv * (ts + 1.0) + th).to(torch.bfloat16).float().numpy()
    assert np.array_equal(O.modulated_norm(v, s, h), want)
    srow = O.bf16_round(rng.standard_normal(W).astype(np.float32))
    hrow = O.bf16_round(rng.standard_normal(W).astype(np.float32))
    sc = torch.from_numpy(srow) + ts
    sh = torch.from_numpy(hrow) + th
    want = (tv * (sc + 1.0) + sh).to(torch.bfloat16).float().numpy()
    assert np.array_equal(O.modulated_norm(v, s, h, srow, hrow), want)


def test_modulated_norm_rounds_the_product_before_the_shift():
    """v = 1 + 2^-12, s = 2^-12, h = -(1 + 2^-11): RN(v·(1 + s)) drops the 2^-24 of the exact
    product (a tie, to even), so the separately rounded result is 0, while a fused
    multiply-add would keep 2^-24."""
    v = np.float32(1 + 2.0 ** -12)
    s = np.float32(2.0 ** -12)
    h = np.float32(-(1 + 2.0 ** -11))
    assert O.modulated_norm(np.array([v]), np.array([s]), np.array([h]))[0] == 0.0
    fused = float(v) * (1 + float(s)) + float(h)
    assert fused == 2.0 ** -24


def test_layer_norm_is_torch_layer_norm():
    """Affine-free LayerNorm with the biased variance: torch's layer_norm in float64."""
    rng = np.random.default_rng(43)
    x = (3 + 2 * rng.standard_normal((5, 7, 1536))).astype(np.float32)
    want = torch.nn.functional.layer_norm(torch.from_numpy(x).double(), (1536,), eps=1e-6).float().numpy()
    np.testing.assert_allclose(O.layer_norm(x, 1e-6), want, rtol=0, atol=2e-7)
    got = O.layer_norm(x, 1e-6).astype(np.float64)
    np.testing.assert_allclose(got.mean(-1), 0, atol=1e-6)
    np.testing.assert_allclose((got ** 2).mean(-1), 1, atol=1e-5)


def test_modulated_norm_backward_is_torch_autograd():
    """The closed-form gradients of LN(x)·(1 + s) + h against torch autograd in float64, for
    the hidden state, the per-element scale and shift, and the row statistics."""
    rng = np.random.default_rng(47)
    B, T, W, eps = 2, 5, 64, 1e-6
    x = 3 + 2 * rng.standard_normal((B, T, W))
    g = rng.standard_normal((B, T, W))
    s = 0.1 * rng.standard_normal((B, T, W))
    srow = 0.1 * rng.standard_normal(W)
    h = 0.1 * rng.standard_normal((B, T, W))
    tx = torch.tensor(x, requires_grad=True)
    ts = torch.tensor(s, requires_grad=True)
    th = torch.tensor(h, requires_grad=True)
    n = torch.nn.functional.layer_norm(tx, (W,), eps=eps)
    out = n * (1 + (torch.tensor(srow) + ts)) + th
    out.backward(torch.tensor(g))
    dx, ds, dh, mean, rstd = O.modulated_norm_backward(x, g, s, eps, srow)
    np.testing.assert_allclose(dx, tx.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(ds, ts.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dh, th.grad.numpy(), rtol=0, atol=0)
    np.testing.assert_allclose(mean, x.mean(-1), rtol=1e-12)
    np.testing.assert_allclose(rstd, 1 / np.sqrt(x.var(-1) + eps), rtol=1e-12)
