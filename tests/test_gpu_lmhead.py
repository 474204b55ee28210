"""GPU: the logits producer (tsm_lm_head) against the oracle's output layer
(rmsnorm, kernels.rs:522-528, then the Bf16 matmul, weights.rs:230-239).

Bar (floating point; the reference's own dot products fold in a
platform-dependent order, so no bit pattern is the target):
  * with TSM_LM_SPLIT every logit within 2^-16 * S of the oracle's, where
    S = sum_k |W[v][k] * xb[r][k]| (f64) bounds the size of any rounding
    of the sum; without it (activations rounded to bf16, relative error up
    to 2^-9 each) within 2^-8 * S;
  * on one-hot weights (a logit is then one activation) within 2^-16 (split)
    or 2^-8 (bf16) of that activation: this pins the MFMA tile layout, the
    vocabulary and row tails, the row stride and the output stride;
  * split error at least 16 times below the bf16 mode's on the same inputs;
  * columns past `vocab` in a wider output row are never written, and two
    calls give identical logits.
A wrong row, column or k index moves a logit by about the size of a whole
dot product, far outside these bounds.
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL_SPLIT = 2.0 ** -16
TOL_BF16 = 2.0 ** -8


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def bf16_bits(a):
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_f64(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def run(x, g, eps, wbits, split, ld=None, x_stride=None):
    """tsm_lm_head through the Python wrapper; x f32 [rows, dim] (host), wbits u16 [vocab, dim]."""
    import torch

    from tachyon_amd.lmhead import lm_head

    rows, dim = x.shape
    vocab = wbits.shape[0]
    xs = x_stride or dim
    xd = torch.zeros(rows, xs, dtype=torch.float32, device="cuda")
    xd[:, :dim] = torch.from_numpy(x).cuda()
    xv = xd[:, :dim]
    gd = torch.from_numpy(np.ascontiguousarray(g, np.float32)).cuda()
    wd = torch.from_numpy(wbits.view(np.int16)).cuda().view(torch.bfloat16)
    out = torch.full((rows, ld or vocab), -7.0, dtype=torch.float32, device="cuda")
    lm_head(xv, gd, eps, wd, split=split, out=out)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def bound_s(wbits, xb):
    return np.abs(xb.astype(np.float64)) @ np.abs(bf16_f64(wbits)).T


def check(case, got, want, s, tol):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    worst = float((err / np.maximum(s, 1e-30)).max())
    say(f"{case}: max |gpu - oracle| / S = {worst:.3g} (bound {tol:.3g}), max abs {float(err.max()):.3g}")
    assert np.all(err <= tol * s + 1e-30), case


@pytest.mark.parametrize("rows", [200, 70, 40, 20])
def test_one_hot_weights_pin_the_layout(oracle, rows):
    """Row v of W picks activation (5v + 3) mod dim: logit (r, v) is then
    xb[r][(5v + 3) mod dim].  Rows 200, 70, 40 and 20 (the 256-, 128-, 64-
    and 32-row workgroup tiles, none a multiple of 16), vocab 333 (not a
    multiple of 128), a row stride of dim + 8 and an output row of vocab + 5
    columns."""
    dim, vocab = 128, 333
    rng = np.random.default_rng(11)
    x = rng.normal(0, 1.5, (rows, dim)).astype(np.float32)
    g = rng.normal(1, 0.2, dim).astype(np.float32)
    w = np.zeros((vocab, dim), np.float32)
    pick = (5 * np.arange(vocab) + 3) % dim
    w[np.arange(vocab), pick] = 1.0
    wb = bf16_bits(w)
    xb = oracle.rmsnorm(x, g, 1e-6)
    want = xb[:, pick]
    for split, tol in ((True, TOL_SPLIT), (False, TOL_BF16)):
        say(f"one-hot rows={rows} dim={dim} vocab={vocab} split={split}")
        got = run(x, g, 1e-6, wb, split, ld=vocab + 5, x_stride=dim + 8)
        assert np.all(got[:, vocab:] == -7.0), "a column past vocab was written"
        err = np.abs(got[:, :vocab].astype(np.float64) - want)
        assert np.all(err <= tol * np.abs(want) + 1e-30), (split, float(err.max()))


@pytest.mark.parametrize("rows,dim,vocab", [(1, 64, 1), (7, 128, 1000), (64, 640, 4099), (100, 192, 700),
                                             (300, 256, 2000), (3, 8192, 500)])
def test_random_against_the_oracle(oracle, rows, dim, vocab):
    rng = np.random.default_rng(rows * 7919 + dim + vocab)
    x = rng.normal(0, 2.0, (rows, dim)).astype(np.float32)
    g = rng.normal(1, 0.3, dim).astype(np.float32)
    wb = bf16_bits(rng.normal(0, 0.05, (vocab, dim)).astype(np.float32))
    want = oracle.lm_head(x, g, 1e-5, wb)
    xb = oracle.rmsnorm(x, g, 1e-5)
    s = bound_s(wb, xb)
    exact = xb.astype(np.float64) @ bf16_f64(wb).T
    errs = {}
    for split, tol in ((True, TOL_SPLIT), (False, TOL_BF16)):
        case = f"random rows={rows} dim={dim} vocab={vocab} split={split}"
        say(case)
        got = run(x, g, 1e-5, wb, split)
        check(case, got, want, s, tol)
        errs[split] = float(np.sqrt(np.mean((got.astype(np.float64) - exact) ** 2)))
    say(f"rms error vs exact: split {errs[True]:.3g}, bf16 {errs[False]:.3g}")
    assert errs[True] * 16 <= errs[False]


def test_full_size_sample(oracle):
    """The bench shape: 256 rows, dim 4096, vocab 151936, checked on a sample
    of 4 rows x 640 vocab ids (among them the last 128, the vocabulary's
    partial tile), and twice in a row for identical results."""
    import torch

    from tachyon_amd.lmhead import lm_head

    rows, dim, vocab = 256, 4096, 151936
    say(f"full size rows={rows} dim={dim} vocab={vocab}")
    gen = torch.Generator(device="cuda").manual_seed(7)
    x = torch.randn(rows, dim, generator=gen, device="cuda", dtype=torch.float32) * 3.0
    g = 1.0 + 0.2 * torch.randn(dim, generator=gen, device="cuda", dtype=torch.float32)
    w = (torch.randn(vocab, dim, generator=gen, device="cuda", dtype=torch.float32) * 0.02).to(torch.bfloat16)
    for split, tol in ((True, TOL_SPLIT), (False, TOL_BF16)):
        out = lm_head(x, g, 1e-6, w, split=split)
        out2 = lm_head(x, g, 1e-6, w, split=split)
        torch.cuda.synchronize()
        assert torch.equal(out, out2), "two calls differ"
        rsel = np.array([0, 97, 200, 255])
        rng = np.random.default_rng(8)
        vsel = np.concatenate([rng.choice(vocab - 128, 512, replace=False), np.arange(vocab - 128, vocab)])
        wb = w[torch.from_numpy(vsel).cuda()].view(torch.int16).cpu().numpy().view(np.uint16)
        xs = x[torch.from_numpy(rsel).cuda()].cpu().numpy()
        gs = g.cpu().numpy()
        want = oracle.lm_head(xs, gs, 1e-6, wb)
        s = bound_s(wb, oracle.rmsnorm(xs, gs, 1e-6))
        got = out[torch.from_numpy(rsel).cuda()][:, torch.from_numpy(vsel).cuda()].cpu().numpy()
        check(f"full size sample split={split}", got, want, s, tol)


def test_logits_feed_the_sampler(oracle):
    """The producer's logits stay on the device and go straight into
    tsm_sample (row stride = vocab): rows with the c4 settings (repetition,
    presence and frequency penalties over a history, top-k, top-p, min-p,
    top-5 logprobs) and plain temperature rows sampled from them equal the
    oracle's sampling of the same logits, copied back, in every token, kept
    count and probability (the sampler's own bar)."""
    import dataclasses

    import torch

    from parity import check
    from tachyon_amd import workloads as wl
    from tachyon_amd.device import Outputs, SamplerContext, upload
    from tachyon_amd.lmhead import lm_head

    rows, dim, vocab = 48, 512, 32000
    say(f"lm_head -> tsm_sample rows={rows} dim={dim} vocab={vocab}")
    gen = torch.Generator(device="cuda").manual_seed(31)
    x = torch.randn(rows, dim, generator=gen, device="cuda", dtype=torch.float32) * 3.0
    g = 1.0 + 0.2 * torch.randn(dim, generator=gen, device="cuda", dtype=torch.float32)
    w = (torch.randn(vocab, dim, generator=gen, device="cuda", dtype=torch.float32) * 0.1).to(torch.bfloat16)
    logits = lm_head(x, g, 1e-6, w, split=True)
    rng = np.random.default_rng(32)
    params = wl.make_params(rows, temperature=0.7, top_k=64, top_p=0.92, repetition_penalty=1.1,
                            presence_penalty=0.4, frequency_penalty=0.2, min_p=0.02, flags=2, n_logprobs=5)
    params[rows // 2:] = wl.make_params(rows - rows // 2, temperature=1.0, top_p=0.95)
    hist = [rng.integers(0, vocab, 128).astype(np.uint32) for _ in range(rows)]
    offs = np.zeros(rows + 1, np.uint32)
    offs[1:] = np.cumsum([len(h) for h in hist])
    host = wl.Workload("lm->sample", logits.cpu().numpy(), vocab, params, np.concatenate(hist), offs, None,
                       wl.uniforms(rng, rows), top_stride=5)
    b = dataclasses.replace(upload(host), logits=logits)  # the producer's own buffer
    ctx = SamplerContext(rows, vocab)
    out = Outputs(rows, 5)
    ctx.sample(b, out)
    torch.cuda.synchronize()
    assert ctx.status() == 0
    check(host, out.numpy(), oracle.sample_batch(host), "lm_head -> tsm_sample")


def test_tile_boundaries(oracle):
    """Rows on both sides of every tile change (32/33, 64/65, 128/129,
    256/257, 513: several 256-row tiles), hidden sizes 896 and 3584 (not
    powers of two) and vocabularies ending one id into, or one id short of,
    a 128-id tile; every logit of every row within the split bound."""
    rng = np.random.default_rng(77)
    shapes = [(32, 896, 129), (33, 896, 255), (64, 192, 128), (65, 192, 383), (128, 3584, 257),
              (129, 128, 1), (256, 64, 640), (257, 64, 641), (513, 128, 300)]
    for rows, dim, vocab in shapes:
        say(f"tile boundary rows={rows} dim={dim} vocab={vocab}")
        x = rng.normal(0, 2.0, (rows, dim)).astype(np.float32)
        g = rng.normal(1, 0.3, dim).astype(np.float32)
        wb = bf16_bits(rng.normal(0, 0.05, (vocab, dim)).astype(np.float32))
        want = oracle.lm_head(x, g, 1e-5, wb)
        s = bound_s(wb, oracle.rmsnorm(x, g, 1e-5))
        check(f"rows={rows} dim={dim} vocab={vocab}", run(x, g, 1e-5, wb, True), want, s, TOL_SPLIT)


def test_seeded_shape_sweep(oracle):
    """Random shapes against the oracle at the bounds above: rows 1-300 (every
    tile), dim a random multiple of 64 up to 2048, vocab 1-3000 (every tail),
    both activation modes, activation widths over a few octaves.
    TSM_LM_SWEEP (environment) sets the number of cases (16)."""
    import os

    cases = int(os.environ.get("TSM_LM_SWEEP", 16))
    for k in range(cases):
        rng = np.random.default_rng(0x1A40 + k)
        rows = int(rng.choice([1, 2, 31, 32, 33, 64, 65, 128, 129, 200, 256, 300]))
        dim = 64 * int(rng.integers(1, 33))
        vocab = int(rng.integers(1, 3001))
        x = (rng.normal(0, 1, (rows, dim)) * np.exp(rng.normal(0, 2))).astype(np.float32)
        g = rng.normal(1, 0.3, dim).astype(np.float32)
        wb = bf16_bits(rng.normal(0, 0.05, (vocab, dim)).astype(np.float32))
        want = oracle.lm_head(x, g, 1e-5, wb)
        s = bound_s(wb, oracle.rmsnorm(x, g, 1e-5))
        split = bool(k % 2)
        case = f"lm sweep case {k}: rows {rows} dim {dim} vocab {vocab} split {split}"
        check(case, run(x, g, 1e-5, wb, split), want, s, TOL_SPLIT if split else TOL_BF16)
