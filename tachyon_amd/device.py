"""Python front end of the GPU sampling path over the C ABI.

PyTorch provides device memory and the stream (plumbing only); all sampling
work runs in the HIP kernels of lib/libtachyon_sampler.so.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib
from .workloads import ROW_PARAMS_DTYPE, Workload


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


@dataclass
class DeviceBatch:
    """A workload's inputs resident in HBM (torch tensors on cuda)."""
    logits: "object"
    usable: int
    params: "object"
    hist_ids: "object"
    hist_offsets: "object"
    mask: "object"
    uniforms: "object"
    top_stride: int
    row_kinds: int = 0          # OR of tsm_row_kind() over the rows (0: not known)
    dist_kinds: int = 0         # the same for tsm_distribution() (masks do not apply)

    @property
    def rows(self):
        return int(self.logits.shape[0])

    @property
    def row_stride(self):
        return int(self.logits.shape[1])

    @property
    def mask_stride(self):
        return 0 if self.mask is None else int(self.mask.shape[1])


SPLIT_ROWS_MAX = 16  # batches of at most this many rows run the split-row kernel


def row_kinds(w: Workload, has_mask: bool) -> int:
    """OR of tsm_row_kind() over the workload's rows, from its host-side
    parameters and history lengths (what a caller knows before the step).
    In a batch small enough for the split-row kernel, a row it takes adds
    only TSM_ROWKIND_SPLIT (its other bit names the whole-row kernel that
    would take it in a larger batch), so no whole-row kernel is queued for
    nothing."""
    L = _lib.lib()
    params = np.ascontiguousarray(w.params)
    hl = np.zeros(w.rows, np.int64) if w.hist_offsets is None else np.diff(w.hist_offsets.astype(np.int64))
    kinds = 0
    base = params.ctypes.data
    small = w.rows <= SPLIT_ROWS_MAX
    for r in range(w.rows):
        k = int(L.tsm_row_kind(ctypes.c_void_p(base + r * params.itemsize), w.usable, int(hl[r]),
                               1 if has_mask else 0))
        kinds |= _lib.ROWKIND_SPLIT if (small and k & _lib.ROWKIND_SPLIT) else k
    return kinds


def upload(w: Workload, device="cuda:0", kinds=True) -> DeviceBatch:
    import torch

    def t(a, dtype=None):
        if a is None:
            return None
        return torch.from_numpy(np.ascontiguousarray(a)).to(device)

    params = torch.from_numpy(np.ascontiguousarray(w.params).view(np.uint8)).to(device)
    return DeviceBatch(
        logits=t(w.logits), usable=w.usable, params=params,
        hist_ids=t(w.hist_ids.view(np.int32)) if w.hist_ids is not None else None,
        hist_offsets=t(w.hist_offsets.view(np.int32)) if w.hist_offsets is not None else None,
        mask=t(w.mask.view(np.int32)) if w.mask is not None else None,
        uniforms=t(w.uniforms), top_stride=max(1, w.top_stride),
        row_kinds=row_kinds(w, w.mask is not None) if kinds else 0,
        dist_kinds=row_kinds(w, False) if kinds else 0)


class Outputs:
    def __init__(self, rows, top_stride, device="cuda:0"):
        import torch

        self.token = torch.zeros(rows, dtype=torch.int32, device=device)
        self.logprob = torch.zeros(rows, dtype=torch.float32, device=device)
        self.top_ids = torch.zeros(rows, top_stride, dtype=torch.int32, device=device)
        self.top_lp = torch.zeros(rows, top_stride, dtype=torch.float32, device=device)
        self.prob = torch.zeros(rows, dtype=torch.float32, device=device)
        self.keep = torch.zeros(rows, dtype=torch.int32, device=device)
        self.top_stride = top_stride

    def numpy(self):
        return dict(
            token=self.token.cpu().numpy().view(np.uint32),
            logprob=self.logprob.cpu().numpy(),
            top_ids=self.top_ids.cpu().numpy().view(np.uint32),
            top_lp=self.top_lp.cpu().numpy(),
            prob=self.prob.cpu().numpy(),
            keep=self.keep.cpu().numpy().view(np.uint32),
        )


class SamplerContext:
    """Owns a tsm_ctx (device scratch sized for max_rows x max_vocab)."""

    def __init__(self, max_rows: int, max_vocab: int, device: int = 0):
        L = _lib.lib()
        err = _lib._err()
        self._h = L.tsm_create(device, max_rows, max_vocab, err, len(err))
        if not self._h:
            raise _lib.TsmError(err.value.decode())
        self.max_rows, self.max_vocab, self.device = max_rows, max_vocab, device

    def close(self):
        if getattr(self, "_h", None):
            _lib.lib().tsm_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown: the library's module state may be gone already
            pass

    def _batch(self, b: DeviceBatch, uniforms=True):
        return _lib.TsmBatch(
            _ptr(b.logits), b.rows, b.row_stride, b.usable, b.mask_stride, _ptr(b.params),
            _ptr(b.hist_ids), _ptr(b.hist_offsets), _ptr(b.mask), _ptr(b.uniforms) if uniforms else None,
            b.row_kinds if uniforms else b.dist_kinds, 0)

    def sample(self, b: DeviceBatch, out: Outputs, stream=None, with_prob=True, with_keep=True,
               with_logprobs=True):
        import torch

        s = stream if stream is not None else torch.cuda.current_stream().cuda_stream
        ob = _lib.TsmOutputs(
            _ptr(out.token), _ptr(out.logprob) if with_logprobs else None,
            _ptr(out.top_ids) if with_logprobs else None, _ptr(out.top_lp) if with_logprobs else None,
            out.top_stride if with_logprobs else 0, 0,
            _ptr(out.prob) if with_prob else None, _ptr(out.keep) if with_keep else None)
        bb = self._batch(b)
        err = _lib._err()
        rc = _lib.lib().tsm_sample(self._h, ctypes.c_void_p(s), ctypes.byref(bb), ctypes.byref(ob), err,
                                   len(err))
        if rc != 0:
            raise _lib.TsmError(err.value.decode())

    def distribution(self, b: DeviceBatch, dist_stride: int, stream=None):
        import torch

        s = stream if stream is not None else torch.cuda.current_stream().cuda_stream
        ids = torch.zeros(b.rows, dist_stride, dtype=torch.int32, device=b.logits.device)
        ps = torch.zeros(b.rows, dist_stride, dtype=torch.float32, device=b.logits.device)
        keep = torch.zeros(b.rows, dtype=torch.int32, device=b.logits.device)
        bb = self._batch(b, uniforms=False)
        err = _lib._err()
        rc = _lib.lib().tsm_distribution(self._h, ctypes.c_void_p(s), ctypes.byref(bb), _ptr(ids), _ptr(ps),
                                         dist_stride, _ptr(keep), err, len(err))
        if rc != 0:
            raise _lib.TsmError(err.value.decode())
        return ids, ps, keep

    def status(self) -> int:
        st = ctypes.c_uint32()
        err = _lib._err()
        if _lib.lib().tsm_status(self._h, ctypes.byref(st), err, len(err)) != 0:
            raise _lib.TsmError(err.value.decode())
        return int(st.value)


def _outputs(out: Outputs):
    return _lib.TsmOutputs(_ptr(out.token), _ptr(out.logprob), _ptr(out.top_ids), _ptr(out.top_lp), out.top_stride,
                           0, _ptr(out.prob), _ptr(out.keep))


def sample_static(b: DeviceBatch, out: Outputs, status=None, stream=None):
    """tsm_sample_static(): one step with no context and no allocation; status
    (an int32 cuda tensor of one element, or None) gets the call's status bits."""
    import torch

    s = stream if stream is not None else torch.cuda.current_stream().cuda_stream
    bb = _lib.TsmBatch(_ptr(b.logits), b.rows, b.row_stride, b.usable, b.mask_stride, _ptr(b.params),
                       _ptr(b.hist_ids), _ptr(b.hist_offsets), _ptr(b.mask), _ptr(b.uniforms), b.row_kinds, 0)
    ob = _outputs(out)
    err = _lib._err()
    rc = _lib.lib().tsm_sample_static(ctypes.c_void_p(s), ctypes.byref(bb), ctypes.byref(ob), _ptr(status), err,
                                      len(err))
    if rc != 0:
        raise _lib.TsmError(err.value.decode())


def run_workload(ctx: SamplerContext, w: Workload, device="cuda:0", kinds=True):
    """Uploads `w`, samples every row on the GPU, returns numpy outputs.
    kinds=False leaves the batch's row kinds unknown (every kernel queued)."""
    import torch

    b = upload(w, device, kinds=kinds)
    out = Outputs(w.rows, max(1, w.top_stride), device)
    ctx.sample(b, out)
    torch.cuda.synchronize()
    return out.numpy()


assert ROW_PARAMS_DTYPE.itemsize == 40
