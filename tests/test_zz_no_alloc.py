"""tsm_sample_static (no context, no allocation) against tsm_sample on the
same inputs, two calls in a row, the second with a smaller batch: results
identical bit for bit, status clear."""
import numpy as np
import pytest

from tachyon_amd import workloads as wl

pytestmark = pytest.mark.gpu


def _compare(ctx, w):
    import torch

    from tachyon_amd.device import Outputs, sample_static, upload

    b = upload(w)
    ref = Outputs(w.rows, max(1, w.top_stride))
    ctx.sample(b, ref)
    got = Outputs(w.rows, max(1, w.top_stride))
    st = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    sample_static(b, got, status=st)
    torch.cuda.synchronize()
    assert ctx.status() == 0
    assert int(st.item()) == 0
    a, c = ref.numpy(), got.numpy()
    for k in a:
        assert np.array_equal(a[k].view(np.uint32), c[k].view(np.uint32)), k
    return a


def test_static_entry_matches_context():
    import torch

    from tachyon_amd.device import SamplerContext

    assert torch.cuda.is_available()
    ctx = SamplerContext(max_rows=256, max_vocab=151936)
    try:
        # a small batch on the split-row kernel (the static scratch), then a
        # smaller one: the scratch keeps nothing between calls
        full = wl.c4()
        sel = np.arange(16)
        w1 = wl.Workload("c4x16", np.ascontiguousarray(full.logits[sel]), full.usable, full.params[sel].copy(),
                         None, None, np.ascontiguousarray(full.mask[sel]), full.uniforms[sel].copy(),
                         top_stride=full.top_stride)
        _compare(ctx, w1)
        _compare(ctx, wl.random_case(seed=77, vocab=9000, rows=5, masked=True))
        # a large batch takes the whole-row kernel (the status word only)
        _compare(ctx, wl.c4(rows=64))
    finally:
        ctx.close()
