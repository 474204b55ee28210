"""GPU: the Q8 logits producer (tsm_lm_head_q8) against the oracle's Q8
output layer: rmsnorm (kernels.rs:522-528), quantize_q8 of each row
(kernels.rs:84-100, as quantize_input, weights.rs:652-664), then the scalar
dot_q8_with (kernels.rs:1420-1430) over Q8Rows (weights.rs:344-374).

Bar: bit-exact, compared as bit patterns.  Every step of the reference's
scalar path fixes its result: the sum of squares is a left fold, each value
is quantized on its own, a block's integer dot is exact (the MFMA sums in
i32), and the blocks' terms (s * wscale) * xscale are added in block order
starting from -0.0.  (The reference's AVX2 and NEON paths add in other
orders and so differ from its own scalar path in the last bits; the GPU
reproduces the scalar one.)  A wrong row, id, block or scale index, a
transposed fragment or a changed rounding shows up as differing bits.
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def weights(rng, vocab, dim):
    wq = rng.integers(-127, 128, (vocab, dim)).astype(np.int8)
    ws = (rng.normal(0, 1, (vocab, dim // 32)) * 0.01).astype(np.float16).view(np.uint16)
    return wq, ws


def run(x, g, eps, wq, ws, ld=None, x_stride=None, calls=1):
    """tsm_lm_head_q8 through the Python wrapper on host arrays; returns each call's logits."""
    import torch

    from tachyon_amd.lmhead import lm_head_q8

    rows, dim = x.shape
    vocab = wq.shape[0]
    xs = x_stride or dim
    xd = torch.zeros(rows, xs, dtype=torch.float32, device="cuda")
    xd[:, :dim] = torch.from_numpy(x).cuda()
    gd = torch.from_numpy(np.ascontiguousarray(g, np.float32)).cuda()
    wqd = torch.from_numpy(wq).cuda()
    wsd = torch.from_numpy(ws.view(np.int16)).cuda()
    outs = []
    for _ in range(calls):
        out = torch.full((rows, ld or vocab), -7.0, dtype=torch.float32, device="cuda")
        lm_head_q8(xd[:, :dim], gd, eps, wqd, wsd, out=out)
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    return outs


def check(case, got, want):
    bad = got.view(np.uint32) != want.view(np.uint32)
    say(f"{case}: {int(bad.sum())} of {bad.size} logits differ in bits")
    if bad.any():
        i, j = np.argwhere(bad)[0]
        raise AssertionError(f"{case}: row {i} id {j}: gpu {got[i, j]!r} oracle {want[i, j]!r}")


@pytest.mark.parametrize("rows,dim,vocab", [(1, 128, 100), (20, 4096, 1000), (40, 160, 515), (100, 96, 700),
                                            (256, 512, 333), (300, 256, 4097), (17, 32, 64), (5, 224, 257),
                                            (3, 4096, 1000), (16, 1024, 4099), (9, 768, 300), (31, 512, 777),
                                            (2, 5120, 300), (40, 8192, 500)])
def test_random_bit_exact(oracle, rows, dim, vocab):
    """Every tile shape (16, 32, 64, 128 and 256 rows; 256, 128 and 64 ids)
    with and without row and vocabulary tails, rows of 1 to 128 blocks, odd
    counts included (the last pair of blocks then has one block), rows
    longer than the prep kernel's 4096-value stage (5120, 8192), and both
    ways of reading the weight scales: 16 pairs at a time (dim a multiple of
    256; for up to 32 rows with whole weight lines through LDS) and 2 bytes
    a pair."""
    rng = np.random.default_rng(rows * 7 + dim + vocab)
    x = rng.normal(0, 1.5, (rows, dim)).astype(np.float32)
    g = rng.normal(1.0, 0.2, dim).astype(np.float32)
    wq, ws = weights(rng, vocab, dim)
    say(f"q8 random rows={rows} dim={dim} vocab={vocab}")
    (got,) = run(x, g, 1e-5, wq, ws)
    check(f"q8 {rows}x{dim}x{vocab}", got, oracle.lm_head_q8(x, g, 1e-5, wq, ws))


def test_strides_and_repeat(oracle):
    """A row stride above dim, an output row wider than the vocabulary (the
    columns past it keep their contents) and two calls with identical bits."""
    rng = np.random.default_rng(3)
    rows, dim, vocab = 40, 256, 200
    x = rng.normal(0, 1, (rows, dim)).astype(np.float32)
    g = rng.normal(1.0, 0.2, dim).astype(np.float32)
    wq, ws = weights(rng, vocab, dim)
    say("q8 strides")
    a, b = run(x, g, 1e-6, wq, ws, ld=263, x_stride=300, calls=2)
    assert np.all(a[:, vocab:] == -7.0)
    check("q8 strides", a[:, :vocab], oracle.lm_head_q8(x, g, 1e-6, wq, ws))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_edge_rows(oracle):
    """Rows the quantization treats specially: all zeros (every block's scale
    is 0, so each logit is a signed zero whose sign follows the weight
    scales), one spike (every other block of the row quantizes to small
    values or 0), values near the f32 limit (the sum of squares overflows to
    infinity, so the normalization factor is 0 and so is the row), a NaN
    (the whole row is NaN after normalization and quantizes to 0), a ramp
    and a row of sign-alternating pairs."""
    rng = np.random.default_rng(4)
    rows, dim, vocab = 8, 256, 300
    x = rng.normal(0, 1, (rows, dim)).astype(np.float32)
    x[0] = 0.0
    x[1] = 1e-3
    x[1, 77] = 50.0
    x[2, :] = 3e38
    x[3, 5] = np.nan
    x[4] = np.tile(np.arange(32, dtype=np.float32) - 15.5, dim // 32)
    x[5, ::2] = -x[5, 1::2]
    g = np.ones(dim, np.float32)
    wq, ws = weights(rng, vocab, dim)
    ws[:7] = 0x8000 | (ws[:7] & 0x7FFF)  # ids 0..6: every scale negative
    say("q8 edge rows")
    (got,) = run(x, g, 1e-5, wq, ws)
    want = oracle.lm_head_q8(x, g, 1e-5, wq, ws)
    check("q8 edge rows", got, want)
    assert np.signbit(got[0, :7]).all()


def test_full_size_rows(oracle):
    """The bench's shape (256 rows, dim 4096, vocab 151936): four rows across
    both ends of the row tiles, every id, bit for bit (each row is quantized
    and summed on its own, so a subset of rows checks the same arithmetic)."""
    import torch

    from tachyon_amd.lmhead import lm_head_q8

    rows, dim, vocab = 256, 4096, 151936
    gen = torch.Generator(device="cuda").manual_seed(8)
    say(f"q8 full size rows={rows} dim={dim} vocab={vocab}")
    x = torch.randn(rows, dim, device="cuda", generator=gen)
    g = 1.0 + 0.1 * torch.randn(dim, device="cuda", generator=gen)
    wq = torch.randint(-127, 128, (vocab, dim), dtype=torch.int8, device="cuda", generator=gen)
    ws = (0.01 * torch.randn(vocab, dim // 32, device="cuda", generator=gen)).to(torch.float16).view(torch.int16)
    out = lm_head_q8(x, g, 1e-6, wq, ws)
    out2 = lm_head_q8(x, g, 1e-6, wq, ws)
    torch.cuda.synchronize()
    pick = [0, 15, 16, 255]
    got = out[pick].cpu().numpy()
    assert torch.equal(out.view(torch.int32), out2.view(torch.int32))
    want = oracle.lm_head_q8(x[pick].cpu().numpy(), g.cpu().numpy(), 1e-6, wq.cpu().numpy(),
                             ws.cpu().numpy().view(np.uint16))
    check("q8 full size", got, want)


@pytest.mark.parametrize("rows", [7, 48])
def test_unaligned_scales_take_the_two_byte_path(oracle, rows):
    """Weight scales 2-byte but not 16-byte aligned (a view one element into
    a buffer) at dim 4096: the kernels read them 2 bytes a pair instead of 16
    pairs at a time (for 7 rows in place of whole weight lines), with the
    same bits."""
    import torch

    from tachyon_amd.lmhead import lm_head_q8

    rng = np.random.default_rng(40 + rows)
    dim, vocab = 4096, 700
    x = rng.normal(0, 1, (rows, dim)).astype(np.float32)
    g = rng.normal(1.0, 0.2, dim).astype(np.float32)
    wq, ws = weights(rng, vocab, dim)
    buf = torch.zeros(vocab * (dim // 32) + 1, dtype=torch.int16, device="cuda")
    buf[1:] = torch.from_numpy(ws.view(np.int16).reshape(-1)).cuda()
    wsd = buf[1:].view(vocab, dim // 32)
    assert wsd.data_ptr() % 16 != 0
    say(f"q8 unaligned scales rows={rows}")
    out = lm_head_q8(torch.from_numpy(x).cuda(), torch.from_numpy(g).cuda(), 1e-5, torch.from_numpy(wq).cuda(), wsd)
    torch.cuda.synchronize()
    check(f"q8 unaligned scales {rows}", out.cpu().numpy(), oracle.lm_head_q8(x, g, 1e-5, wq, ws))


def test_seeded_shape_sweep(oracle):
    """Random shapes, bit for bit: rows 1-300 (every tile), dim a random
    multiple of 32 up to 2048 (both ways of reading the weight scales), vocab
    1-3000 (every tail), scales 16-byte aligned or not, random activation
    widths.  TSM_Q8_SWEEP (environment) sets the number of cases (24)."""
    import os

    import torch

    from tachyon_amd.lmhead import lm_head_q8

    cases = int(os.environ.get("TSM_Q8_SWEEP", 24))
    for k in range(cases):
        rng = np.random.default_rng(0x0880 + k)
        rows = int(rng.choice([1, 2, 7, 16, 17, 31, 32, 33, 64, 65, 128, 129, 256, 300]))
        dim = 32 * int(rng.integers(1, 65))
        vocab = int(rng.integers(1, 3001))
        x = (rng.normal(0, 1, (rows, dim)) * np.exp(rng.normal(0, 2))).astype(np.float32)
        g = rng.normal(1.0, 0.3, dim).astype(np.float32)
        wq, ws = weights(rng, vocab, dim)
        off = int(rng.integers(0, 2))
        buf = torch.zeros(vocab * (dim // 32) + off, dtype=torch.int16, device="cuda")
        buf[off:] = torch.from_numpy(ws.view(np.int16).reshape(-1)).cuda()
        wsd = buf[off:].view(vocab, dim // 32)
        out = lm_head_q8(torch.from_numpy(x).cuda(), torch.from_numpy(g).cuda(), 1e-5, torch.from_numpy(wq).cuda(),
                         wsd)
        torch.cuda.synchronize()
        check(f"q8 sweep case {k}: rows {rows} dim {dim} vocab {vocab} scale offset {off}", out.cpu().numpy(),
              oracle.lm_head_q8(x, g, 1e-5, wq, ws))
