"""GPU parity: device generator, scalar math, dequantisation and the affine
QMV against the CPU oracle (bit-exact: the kernel and the oracle share one
fixed operation order), plus closed-form tolerance and batch invariance."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def dev_q(mx, n, k, bits, gs, seed):
    return mx.QWeight.random(n, k, bits, gs, seed)


def test_device_generator_matches_oracle(mx, orc):
    d = mx.DeviceArray(100003, np.uint16)
    for dist, a, b in [(0, 0.005, 0.03), (0, -0.2, 0.2), (1, 1.0, 0.0), (1, 0.5, -1.0)]:
        mx.fill_bf16(d, 42 + dist, dist, a, b)
        assert (d.numpy() == orc.fill_bf16(100003, 42 + dist, dist, a, b)).all()
    for bits in (4, 5, 6, 8):
        w = mx.QWeight.random(37, 512, bits, 64, seed=9 + bits)
        c, s, b = orc.random_qweight(37, 512, bits, 64, seed=9 + bits)
        hc, hs, hb = w.host()
        assert (hc == c).all() and (hs == s).all() and (hb == b).all()


def test_device_math_matches_oracle_bitwise(mx, orc):
    rng = np.random.default_rng(0)
    x = np.concatenate([
        np.linspace(-110, 95, 400001, dtype=np.float32),
        rng.standard_normal(200000).astype(np.float32) * 4,
        np.geomspace(1e-38, 1e3, 100000).astype(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 88.72, -103.97], np.float32),
    ])
    dx = mx.DeviceArray.from_numpy(x)
    dy = mx.DeviceArray(x.shape, np.float32)
    for op in range(5):
        inp = np.abs(x) if op == 1 else x
        dx.upload(inp)
        mx.check(mx.lib.mx_eval_math(op, dx.ptr, dy.ptr, x.size, None))
        got = dy.numpy()
        want = orc.eval_math(op, inp)
        same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
        assert same.all(), (op, inp[~same][:5], got[~same][:5], want[~same][:5])


@pytest.mark.parametrize("bits", [4, 5, 6, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("k,n", [(512, 48), (2560, 640), (256, 72), (1024, 1000)])
def test_qmv_bit_exact(mx, orc, bits, gs, k, n):
    seed = bits * 1000 + gs * 10 + k
    w = dev_q(mx, n, k, bits, gs, seed)
    codes, s, b = orc.random_qweight(n, k, bits, gs, seed)
    for m in (1, 2, 3, 4, 8):
        x = orc.fill_bf16(m * k, seed + m, 1, 1.0, 0.0).reshape(m, k)
        dx = mx.DeviceArray.from_numpy(x)
        dy = mx.DeviceArray((m, n), np.uint16)
        mx.qmv(w, dx, m, dy)
        got = dy.numpy()
        want = orc.qmv(codes, s, b, k, bits, gs, x)
        assert (got == want).all(), (bits, gs, k, n, m, np.argwhere(got != want)[:5])


def test_qmv_config0_exact_and_closed_form(mx, orc):
    """benchmark config 0: x bf16 [1,2048] ~ N(0,1); W [4096,2048] 4-bit g64."""
    n, k, bits, gs = 4096, 2048, 4, 64
    w = dev_q(mx, n, k, bits, gs, 100)
    codes, s, b = orc.random_qweight(n, k, bits, gs, 100)
    x = orc.fill_bf16(k, 101, 1, 1.0, 0.0).reshape(1, k)
    dx = mx.DeviceArray.from_numpy(x)
    dy = mx.DeviceArray((1, n), np.uint16)
    mx.qmv(w, dx, 1, dy)
    got = dy.numpy()
    assert (got == orc.qmv(codes, s, b, k, bits, gs, x)).all()
    y64 = orc.qmv_f64(codes, s, b, k, bits, gs, x)
    g = orc.bf16_to_f32(got).astype(np.float64)
    # north-star tolerance for bf16 outputs: 2e-2 relative / 1e-2 absolute
    assert (np.abs(g - y64) <= 1e-2 + 2e-2 * np.abs(y64)).all()


def test_qmv_batch_rows_equal_single_rows(mx, orc):
    """Row batching never changes a row's bits (reference batch-parity.rs:144-151)."""
    n, k, bits, gs = 1536, 4096, 5, 64
    w = dev_q(mx, n, k, bits, gs, 7)
    x = orc.fill_bf16(8 * k, 8, 1, 1.0, 0.0).reshape(8, k)
    dx = mx.DeviceArray.from_numpy(x)
    dy = mx.DeviceArray((8, n), np.uint16)
    mx.qmv(w, dx, 8, dy)
    batched = dy.numpy()
    for r in range(8):
        d1 = mx.DeviceArray.from_numpy(x[r:r + 1])
        y1 = mx.DeviceArray((1, n), np.uint16)
        mx.qmv(w, d1, 1, y1)
        assert (y1.numpy()[0] == batched[r]).all()


def test_qmv_vocab_head_shape(mx, orc):
    """8-bit head [151936, 2048] at two rows."""
    n, k, bits, gs = 151936, 2048, 8, 64
    w = dev_q(mx, n, k, bits, gs, 55)
    codes, s, b = orc.random_qweight(n, k, bits, gs, 55)
    x = orc.fill_bf16(2 * k, 56, 1, 1.0, 0.0).reshape(2, k)
    dx = mx.DeviceArray.from_numpy(x)
    dy = mx.DeviceArray((2, n), np.uint16)
    mx.qmv(w, dx, 2, dy)
    assert (dy.numpy() == orc.qmv(codes, s, b, k, bits, gs, x)).all()


@pytest.mark.parametrize("bits", [4, 5, 6, 8])
def test_dequant_rows_bit_exact(mx, orc, bits):
    n, k, gs = 3000, 2048, 64
    w = dev_q(mx, n, k, bits, gs, 300 + bits)
    codes, s, b = orc.random_qweight(n, k, bits, gs, 300 + bits)
    ids = np.array([0, 2999, 17, 17, 1234, 5, 2048, 999], np.uint32)
    did = mx.DeviceArray.from_numpy(ids)
    out = mx.DeviceArray((ids.size, k), np.uint16)
    mx.dequant_rows(w, did, ids.size, out)
    assert (out.numpy() == orc.dequant_rows(codes, s, b, k, bits, gs, ids)).all()
