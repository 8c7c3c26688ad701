"""GPU parity of the BitLinear layer entry points (kore_hip_bit_linear_f32 /
_i8): the reference's BitLinear::forward (crates/kore-nn/src/bit_linear.rs:
175-237) is transpose(x) -> ternary_matmul -> transpose -> add(bias); the
device computes it in one launch, reading the layer's input as stored and
writing the output in the layer's [batch, out] layout.

Bar: bit-exact.  Against the oracle's composition of that chain
(oracle.bit_linear_forward / bit_linear_i8) wherever the CPU oracle finishes
in seconds; at the full FFN shape with 4096 tokens, against an f64 GEMM of the
decoded trits (exact for the int8 path's integer sums) and against the
device's own ternary matmuls -- themselves checked bit-exact against the
oracle -- composed with exact transposes and f32 bias adds, plus the oracle
on a slice of tokens.
"""
import sys

import numpy as np
import pytest

import oracle
from inputs import assert_bitexact, int8_codes, normal, prequant_inputs, raw_packed, ternary_weights

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from kore_amd import rocm  # noqa: E402
from kore_amd.rocm import HipBuffer  # noqa: E402

DEV = 0


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def up(arr) -> HipBuffer:
    return HipBuffer.from_host(DEV, np.ascontiguousarray(arr))


def down(buf: HipBuffer, dtype, shape):
    return buf.to_host(dtype)[: int(np.prod(shape))].reshape(shape)


def _offset_buffer(arr: np.ndarray, offset: int) -> HipBuffer:
    """Device copy of arr starting `offset` bytes past a 16-byte boundary."""
    t = torch.empty(arr.nbytes + offset, dtype=torch.uint8, device="cuda")
    t[offset:].copy_(torch.from_numpy(np.ascontiguousarray(arr).view(np.uint8).ravel()))
    return HipBuffer.from_tensor(t[offset:])


def test_bit_linear_reference_kats_on_device():
    """bit_linear.rs tests on the device, weights packed by
    kore_hip_pack_weights_ternary: test_bit_linear_approximates_linear gives
    exactly [3, 4]; test_bit_linear_bias gives [11, 21]; with and without a
    bias through both entry points."""
    w = np.array([[1.0, -1.0, 0.0, 1.0], [-1.0, 1.0, 1.0, 0.0]], np.float32)
    p, s = rocm.rocm_pack_weights_ternary(DEV, up(w), 2, 4, 0.3)
    y = rocm.rocm_bit_linear_f32(DEV, p, s, up(np.array([[1.0, 2.0, 3.0, 4.0]], np.float32)), None, 2, 1, 4)
    assert down(y, np.float32, (1, 2)).tolist() == [[3.0, 4.0]]
    p, s = rocm.rocm_pack_weights_ternary(DEV, up(np.eye(2, dtype=np.float32)), 2, 2, 0.3)
    bias = up(np.array([10.0, 20.0], np.float32))
    y = rocm.rocm_bit_linear_f32(DEV, p, s, up(np.ones((1, 2), np.float32)), bias, 2, 1, 2)
    assert down(y, np.float32, (1, 2)).tolist() == [[11.0, 21.0]]
    # the int8 layer on codes of [1, 1] (scale 1/127 per code 127)
    q = up(np.array([[127, 127]], np.int8))
    qs = up(np.array([1.0 / 127.0], np.float32))
    y = rocm.rocm_bit_linear_i8(DEV, p, s, q, qs, bias, 2, 1, 2)
    want = oracle.bit_linear_i8(down(p, np.uint8, (2, 1)), down(s, np.float32, (2,)), np.array([[127, 127]], np.int8),
                                np.array([1.0 / 127.0], np.float32), np.array([10.0, 20.0], np.float32), 2, 1, 2)
    assert_bitexact(down(y, np.float32, (1, 2)), want, "bit_linear_i8 KAT")


@pytest.mark.parametrize("batch", [1, 64, 4096])
def test_bit_linear_f32_layer_ffn_shape(batch):
    """BitLinear 2560 -> 6912 (the pre-quant config's width) on 1, 64 and
    4096 tokens, with a bias: bit-exact against the oracle's composition
    (all tokens at 1 and 64; the first 8 and the last token at 4096, plus
    every token against the device's ternary_matmul_f32 on x^T transposed
    back, + bias)."""
    m, k = 6912, 2560
    log(f"bit_linear_f32 m={m} batch={batch} k={k}")
    p, sa = ternary_weights(m, k, 31)
    x = normal((batch, k), 32)
    bias = normal((m,), 33)
    bp, bs, bx, bb = up(p), up(sa), up(x), up(bias)
    got = down(rocm.rocm_bit_linear_f32(DEV, bp, bs, bx, bb, m, batch, k), np.float32, (batch, m))
    if batch <= 64:
        assert_bitexact(got, oracle.bit_linear_forward(p, sa, x, bias, m, batch, k), f"bit_linear_f32 batch={batch}")
        return
    for rows in (slice(0, 8), slice(batch - 1, batch)):
        xs = x[rows]
        assert_bitexact(got[rows], oracle.bit_linear_forward(p, sa, xs, bias, m, xs.shape[0], k),
                        f"bit_linear_f32 batch={batch} tokens {rows}")
    xt = torch.from_numpy(x).cuda().t().contiguous()
    c = rocm.rocm_ternary_matmul_f32(DEV, bp, bs, HipBuffer.from_tensor(xt), m, batch, k)
    ct = torch.from_numpy(down(c, np.float32, (m, batch))).cuda()
    want = ct.t().contiguous() + torch.from_numpy(bias).cuda()[None, :]
    assert torch.equal(torch.from_numpy(got).cuda(), want), "bit_linear_f32 vs ternary_matmul_f32 composition"


@pytest.mark.parametrize("batch", [1, 64, 4096])
def test_bit_linear_i8_layer_ffn_shape(batch):
    """Pre-quant -> BitLinear 2560 -> 6912 on 1, 64 and 4096 tokens, with a
    bias: the codes of kore_hip_rms_norm_quant_i8 fed to kore_hip_bit_linear_i8;
    bit-exact against the oracle's composition (1 and 64 tokens; a slice at
    4096) and against an f64 GEMM of the decoded trits and codes (exact) with
    the f32 epilogue, transposed, + bias (every token)."""
    m, k = 6912, 2560
    log(f"bit_linear_i8 m={m} batch={batch} k={k}")
    p, sa = ternary_weights(m, k, 34)
    x, g = prequant_inputs(batch, k, 0)
    bias = normal((m,), 35)
    qb, sb = rocm.rocm_rms_norm_quant_i8(DEV, up(x), up(g), batch, k, 1e-6)
    bp, bs, bb = up(p), up(sa), up(bias)
    got = down(rocm.rocm_bit_linear_i8(DEV, bp, bs, qb, sb, bb, m, batch, k), np.float32, (batch, m))
    q = down(qb, np.int8, (batch, k))
    qs = down(sb, np.float32, (batch,))
    if batch <= 64:
        assert_bitexact(got, oracle.bit_linear_i8(p, sa, q, qs, bias, m, batch, k), f"bit_linear_i8 batch={batch}")
    else:
        rows = slice(0, 4)
        assert_bitexact(got[rows], oracle.bit_linear_i8(p, sa, q[rows], qs[rows], bias, m, 4, k),
                        f"bit_linear_i8 batch={batch} first tokens")
    t = torch.from_numpy(oracle.unpack_trits(p, k)).cuda().double()
    acc = (t @ torch.from_numpy(q).cuda().double().T).float()
    c = (acc * torch.from_numpy(sa).cuda()[:, None]) * torch.from_numpy(qs).cuda()[None, :]
    want = c.t().contiguous() + torch.from_numpy(bias).cuda()[None, :]
    assert torch.equal(torch.from_numpy(got).cuda(), want), f"bit_linear_i8 batch={batch} vs f64 GEMM"


def test_bit_linear_i8_down_projection_shape():
    """FFN down-projection 6912 -> 2560 on 4096 tokens (1383-byte packed rows,
    256 x 192 wide tiles) through the layer entry point, no bias: bit-exact
    against an f64 GEMM of the decoded trits, transposed."""
    m, n, k = 2560, 4096, 6912
    log(f"bit_linear_i8 down-projection m={m} n={n} k={k}")
    p, sa = ternary_weights(m, k, 36)
    q = int8_codes(n, k, 37)
    sq = np.abs(normal((n,), 38, 0.02, 0.005))
    got = down(rocm.rocm_bit_linear_i8(DEV, up(p), up(sa), up(q), up(sq), None, m, n, k), np.float32, (n, m))
    t = torch.from_numpy(oracle.unpack_trits(p, k)).cuda().double()
    acc = (t @ torch.from_numpy(q).cuda().double().T).float()
    c = (acc * torch.from_numpy(sa).cuda()[:, None]) * torch.from_numpy(sq).cuda()[None, :]
    assert torch.equal(torch.from_numpy(got).cuda(), c.t().contiguous()), "down-projection layer vs f64 GEMM"


# (m, batch, k): every kernel of both layers -- i8: small-n (batch <= 8), skinny
# (<= 64), 128 x 128 tiles with and without split K, wide tiles of 256 and 192
# columns, code rows that are not 16-byte aligned (k % 16 != 0), the
# one-thread-per-output kernel (k % 8 != 0 at small batch); f32: the fold-wave
# kernel (1-4 tokens), the row-broadcast kernel in 16/32/64-token tiles with a
# partial last K chunk (k % 80 != 0), the per-lane kernel (tiny matrices);
# outputs whose rows are not a multiple of 4 floats.
LAYER_SHAPES = [(7, 1, 25), (130, 2, 1000), (257, 3, 2563), (64, 4, 8), (300, 5, 1203), (6912, 8, 2560),
                (1001, 16, 640), (555, 33, 1283), (2560, 64, 6912), (4100, 300, 560), (1000, 1000, 1001),
                (3333, 3900, 80), (4096, 3072, 640), (2560, 3901, 1280), (4099, 2050, 336), (3, 1, 4), (5, 9, 3)]


def _i8_want(p, sa, q, qs, bias, k):
    """((float)acc * sa) * qs transposed, + bias, on the device: acc from an
    f64 GEMM of the decoded trits and codes (exact integer sums)."""
    t = torch.from_numpy(oracle.unpack_trits(p, k)).cuda().double()
    acc = (t @ torch.from_numpy(q).cuda().double().T).float()
    c = (acc * torch.from_numpy(sa).cuda()[:, None]) * torch.from_numpy(qs).cuda()[None, :]
    y = c.t().contiguous()
    return y + torch.from_numpy(bias).cuda()[None, :] if bias is not None else y


@pytest.mark.parametrize("m,batch,k", LAYER_SHAPES)
def test_bit_linear_layers_every_kernel(m, batch, k):
    """Both layer entry points at shapes that reach every kernel, with and
    without a bias, on arbitrary packed bytes (bytes >= 243 included):
    bit-exact against the oracle's composition on the tokens the CPU oracle
    finishes in seconds, and on every token against an f64 GEMM (int8 layer)
    or the device's ternary_matmul_f32 on x^T (f32 layer), transposed, + bias."""
    log(f"bit_linear layers m={m} batch={batch} k={k}")
    p = raw_packed(m, k, m + 7 * k)
    sa = normal((m,), 40, 1.0, 0.1)
    bias = normal((m,), 41)
    q = int8_codes(batch, k, batch + 3)
    qs = np.abs(normal((batch,), 42, 0.02, 0.005))
    x = normal((batch, k), 43)
    bp, bs, bbias = up(p), up(sa), up(bias)
    tok = slice(0, min(batch, max(1, 300_000_000 // max(1, m * k))))
    xt = torch.from_numpy(x).cuda().t().contiguous()
    c = rocm.rocm_ternary_matmul_f32(DEV, bp, bs, HipBuffer.from_tensor(xt), m, batch, k)
    cf = torch.from_numpy(down(c, np.float32, (m, batch))).cuda().t().contiguous()
    for with_bias in (True, False):
        b_np = bias if with_bias else None
        b_dev = bbias if with_bias else None
        y8 = down(rocm.rocm_bit_linear_i8(DEV, bp, bs, up(q), up(qs), b_dev, m, batch, k), np.float32, (batch, m))
        assert_bitexact(y8[tok], oracle.bit_linear_i8(p, sa, q[tok], qs[tok], b_np, m, q[tok].shape[0], k),
                        f"bit_linear_i8 bias={with_bias}")
        assert torch.equal(torch.from_numpy(y8).cuda(), _i8_want(p, sa, q, qs, b_np, k)), \
            f"bit_linear_i8 bias={with_bias} vs f64 GEMM"
        yf = down(rocm.rocm_bit_linear_f32(DEV, bp, bs, up(x), b_dev, m, batch, k), np.float32, (batch, m))
        xs = x[tok]
        assert_bitexact(yf[tok], oracle.bit_linear_forward(p, sa, xs, b_np, m, xs.shape[0], k),
                        f"bit_linear_f32 bias={with_bias}")
        want = cf + torch.from_numpy(bias).cuda()[None, :] if with_bias else cf
        assert torch.equal(torch.from_numpy(yf).cuda(), want), f"bit_linear_f32 bias={with_bias} vs composition"


@pytest.mark.parametrize("off", [4, 8, 12])
def test_bit_linear_unaligned_buffers(off):
    """Input, codes and output at 4/8/12 bytes past a 16-byte boundary (the
    vector stores fall back to element stores, the token-major loads stay
    in bounds): bit-exact against the oracle's composition."""
    m, batch, k = 4096, 320, 480
    log(f"bit_linear unaligned off={off} m={m} batch={batch} k={k}")
    p, sa = ternary_weights(m, k, 44)
    bias = normal((m,), 45)
    x = normal((batch, k), 46)
    q = int8_codes(batch, k, 47)
    qs = np.abs(normal((batch,), 48, 0.02, 0.005))
    yt = torch.full((batch * m + 4,), float("nan"), dtype=torch.float32, device="cuda")
    yb = HipBuffer.from_tensor(yt[off // 4:])
    rocm.rocm_bit_linear_i8(DEV, up(p), up(sa), _offset_buffer(q, off), up(qs), up(bias), m, batch, k, out=yb)
    torch.cuda.synchronize()
    assert_bitexact(yt[off // 4: off // 4 + batch * m].cpu().numpy().reshape(batch, m),
                    oracle.bit_linear_i8(p, sa, q, qs, bias, m, batch, k), "bit_linear_i8 unaligned")
    yt.fill_(float("nan"))
    rocm.rocm_bit_linear_f32(DEV, up(p), up(sa), _offset_buffer(x, off), up(bias), m, batch, k, out=yb)
    torch.cuda.synchronize()
    got = yt[off // 4: off // 4 + batch * m].cpu().numpy().reshape(batch, m)
    assert_bitexact(got[:16], oracle.bit_linear_forward(p, sa, x[:16], bias, m, 16, k), "bit_linear_f32 unaligned")
    assert torch.isnan(yt[:off // 4]).all() and torch.isnan(yt[off // 4 + batch * m:]).all()


@pytest.mark.parametrize("m,batch,k", [(4097, 48, 2563), (2049, 130, 2605), (1500, 192, 6912), (4100, 41, 2560),
                                       (6000, 64, 3201), (4100, 64, 6917), (2560, 64, 6912), (2600, 41, 2561)])
def test_bit_linear_f32_matrix_core_decode_batches(m, batch, k):
    """The 4 x 4 x 1 matrix-core kernel that takes the f32 layer at 41-192
    tokens (token-major input; K >= 2560 and at least 640 waves of 4 rows x
    64 tokens): ragged row groups (m % 4 == 1, where the packed matrix ends
    inside a dword), partial last column tiles, K not a multiple of the
    80-column chunk or of 5, 6912 columns of packed rows held in LDS; with Inf, NaN and subnormal inputs in some tokens (their
    chunks fold element by element, zero trits skipped).  Bit-exact against
    the oracle's composition on the tokens it finishes in seconds and against
    the device's ternary_matmul_f32 on x^T (another kernel) on every token."""
    log(f"bit_linear_f32 4x4 matrix cores m={m} batch={batch} k={k}")
    p = raw_packed(m, k, 5 * m + k)
    sa = normal((m,), 50, 1.0, 0.1)
    bias = normal((m,), 51)
    x = normal((batch, k), 52)
    r = np.random.default_rng(m + batch)
    x[1, r.integers(0, k, 3)] = np.inf
    x[2, r.integers(0, k, 2)] = -np.inf
    x[3, r.integers(0, k, 2)] = np.nan
    x[4] = (x[4] * 1e-39).astype(np.float32)  # subnormal
    bp, bs, bb = up(p), up(sa), up(bias)
    got = down(rocm.rocm_bit_linear_f32(DEV, bp, bs, up(x), bb, m, batch, k), np.float32, (batch, m))
    tok = slice(0, min(batch, max(8, 100_000_000 // max(1, m * k))))
    xs = x[tok]
    assert_bitexact(got[tok], oracle.bit_linear_forward(p, sa, xs, bias, m, xs.shape[0], k),
                    "bit_linear_f32 4x4 matrix cores vs oracle")
    xt = torch.from_numpy(x).cuda().t().contiguous()
    c = rocm.rocm_ternary_matmul_f32(DEV, bp, bs, HipBuffer.from_tensor(xt), m, batch, k)
    ct = torch.from_numpy(down(c, np.float32, (m, batch))).cuda()
    want = ct.t().contiguous() + torch.from_numpy(bias).cuda()[None, :]
    gt = torch.from_numpy(got).cuda()
    same = (gt == want) | (torch.isnan(gt) & torch.isnan(want))
    assert bool(same.all()), f"bit_linear_f32 4x4 matrix cores vs ternary_matmul_f32: {int((~same).sum())} differ"


@pytest.mark.parametrize("m,batch,k", [(2049, 520, 1284), (1100, 1040, 3200), (4096, 770, 2560),
                                       (13824, 40, 2560), (3000, 24, 1283), (2500, 12, 3203)])
def test_bit_linear_f32_prefill_nonfinite(m, batch, k):
    """The kernels that load the layer's token-major input straight into LDS
    and find Inf/NaN from the sums after each chunk (the chunk refolded with
    zero trits skipped): the 16 x 16 matrix-core kernel (K a multiple of 4)
    and the row-broadcast kernel in 64-, 32- and 16-column tiles (7, 2 and 2
    rows per lane; partial last chunks).  Tokens with Inf, -Inf, NaN,
    subnormal and overflowing inputs, bit-exact against the oracle on those
    tokens and against ternary_matmul_f32 on x^T (other staging) on every
    token."""
    log(f"bit_linear_f32 LDS-loaded input, non-finite m={m} batch={batch} k={k}")
    p = raw_packed(m, k, 3 * m + k)
    sa = normal((m,), 90, 1.0, 0.1)
    bias = normal((m,), 91)
    x = normal((batch, k), 92)
    r = np.random.default_rng(m + batch + k)
    x[0, r.integers(0, k, 2)] = np.inf
    x[1, r.integers(0, k, 3)] = -np.inf
    x[2, r.integers(0, k, 1)] = np.nan
    x[3] = (x[3] * 1e-39).astype(np.float32)  # subnormal
    x[4] = np.float32(3e38)  # the sums overflow
    x[batch - 1, k - 1] = np.nan  # the last chunk of the last token
    bp, bs, bb = up(p), up(sa), up(bias)
    got = down(rocm.rocm_bit_linear_f32(DEV, bp, bs, up(x), bb, m, batch, k), np.float32, (batch, m))
    rows = [0, 1, 2, 3, 4, 5, batch - 1]
    xs = x[rows]
    assert_bitexact(got[rows], oracle.bit_linear_forward(p, sa, xs, bias, m, len(rows), k),
                    "bit_linear_f32 16x16 non-finite vs oracle")
    xt = torch.from_numpy(x).cuda().t().contiguous()
    c = rocm.rocm_ternary_matmul_f32(DEV, bp, bs, HipBuffer.from_tensor(xt), m, batch, k)
    ct = torch.from_numpy(down(c, np.float32, (m, batch))).cuda()
    want = ct.t().contiguous() + torch.from_numpy(bias).cuda()[None, :]
    gt = torch.from_numpy(got).cuda()
    same = (gt == want) | (torch.isnan(gt) & torch.isnan(want))
    assert bool(same.all()), f"bit_linear_f32 16x16 vs ternary_matmul_f32: {int((~same).sum())} differ"


@pytest.mark.parametrize("seed", range(6))
def test_bit_linear_f32_matrix_core_random_shapes(seed):
    """Random shapes across the 4 x 4 x 1 kernel's range (41-192 tokens,
    2560-7680 input features, at least 1024 waves): bit-exact against the oracle on the
    first tokens and against ternary_matmul_f32 on x^T (the row-broadcast or
    16 x 16 kernel, never this one) on every token."""
    r = np.random.default_rng(1000 + seed)
    batch = int(r.integers(41, 193))
    tiles = (batch + 63) // 64
    m = int(r.integers(4096 // tiles, 4096 // tiles + 2000))  # at least 1024 waves of 4 rows x 64 tokens
    k = int(r.integers(2560, 7681))
    log(f"bit_linear_f32 4x4 random seed={seed} m={m} batch={batch} k={k}")
    p = raw_packed(m, k, 11 * seed + 3)
    sa = normal((m,), 60 + seed, 1.0, 0.1)
    bias = normal((m,), 70 + seed) if seed % 2 == 0 else None
    x = normal((batch, k), 80 + seed)
    bp, bs = up(p), up(sa)
    bb = up(bias) if bias is not None else None
    got = down(rocm.rocm_bit_linear_f32(DEV, bp, bs, up(x), bb, m, batch, k), np.float32, (batch, m))
    tok = slice(0, min(batch, max(2, 50_000_000 // max(1, m * k))))
    xs = x[tok]
    assert_bitexact(got[tok], oracle.bit_linear_forward(p, sa, xs, bias, m, xs.shape[0], k),
                    f"bit_linear_f32 4x4 random seed={seed}")
    xt = torch.from_numpy(x).cuda().t().contiguous()
    c = rocm.rocm_ternary_matmul_f32(DEV, bp, bs, HipBuffer.from_tensor(xt), m, batch, k)
    want = torch.from_numpy(down(c, np.float32, (m, batch))).cuda().t().contiguous()
    if bias is not None:
        want = want + torch.from_numpy(bias).cuda()[None, :]
    assert torch.equal(torch.from_numpy(got).cuda(), want), f"bit_linear_f32 4x4 random seed={seed} vs composition"
