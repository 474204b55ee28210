"""The logits producer: Tachyon's output layer on the GPU (tsm_lm_head).

`lm_head(x, norm_w, eps, w)` is the reference's

    rmsnorm(&mut xb, &x[row], &w.norm, eps)      # model.rs:702-709
    head.matmul(pool, &xb, n, &mut logits)       # model.rs:711-715

for a Bf16 lm_head (weights.rs:230-239): x is f32 [rows, dim] (the logit
rows of the batch), norm_w f32 [dim], w the bf16 matrix [vocab, dim]; the
result is f32 [rows, vocab], in the layout tsm_sample reads.  One prep
kernel (the rmsnorm, the bf16 operands) and one MFMA GEMM, both through the
C ABI; torch only holds the device memory and names the stream.  There is
no CPU fallback.
"""
from __future__ import annotations

from . import _lib


def workspace_bytes(rows: int, dim: int, split: bool = True) -> int:
    return int(_lib.lib().tsm_lm_head_workspace(rows, dim, _lib.LM_SPLIT if split else 0))


def lm_head(x, norm_w, eps: float, w, split: bool = True, out=None, workspace=None, stream=None):
    """Logits of the rows of x (see the module docstring).  `split` carries
    each activation as two bf16 values (about f32 accuracy, twice the matrix
    work); without it the activations are rounded to bf16."""
    import torch

    if x.dtype != torch.float32 or norm_w.dtype != torch.float32 or w.dtype != torch.bfloat16:
        raise TypeError("x and norm_w must be float32, w bfloat16")
    if not (x.is_cuda and norm_w.is_cuda and w.is_cuda):
        raise ValueError("x, norm_w and w must be on the GPU")
    if x.dim() != 2 or x.stride(1) != 1 or w.dim() != 2 or not w.is_contiguous() or not norm_w.is_contiguous():
        raise ValueError("x must be [rows, dim] with unit column stride; w [vocab, dim] and norm_w contiguous")
    rows, dim = x.shape
    vocab = w.shape[0]
    if w.shape[1] != dim or norm_w.numel() != dim:
        raise ValueError(f"shapes disagree: x {tuple(x.shape)}, norm_w {tuple(norm_w.shape)}, w {tuple(w.shape)}")
    flags = _lib.LM_SPLIT if split else 0
    need = workspace_bytes(rows, dim, split)
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    if out is None:
        out = torch.empty(rows, vocab, dtype=torch.float32, device=x.device)
    if (out.dtype != torch.float32 or out.dim() != 2 or out.stride(1) != 1 or out.shape[0] < rows
            or out.shape[1] < vocab or not out.is_cuda):
        raise ValueError("out must be float32 [>= rows, >= vocab] on the GPU with unit column stride")
    if workspace.numel() * workspace.element_size() < need or not workspace.is_cuda:
        raise ValueError(f"workspace must hold {need} bytes on the GPU")
    err = _lib._err()
    s = stream if stream is not None else torch.cuda.current_stream().cuda_stream
    rc = _lib.lib().tsm_lm_head(s, x.data_ptr(), x.stride(0), norm_w.data_ptr(), float(eps), w.data_ptr(), rows, dim,
                                vocab, flags, workspace.data_ptr(), workspace.numel() * workspace.element_size(),
                                out.data_ptr(), out.stride(0), err, len(err))
    if rc != 0:
        raise _lib.TsmError(err.value.decode())
    return out


def workspace_bytes_q8(rows: int, dim: int) -> int:
    return int(_lib.lib().tsm_lm_head_q8_workspace(rows, dim))


def lm_head_q8(x, norm_w, eps: float, wq, wscale, out=None, workspace=None, stream=None):
    """Logits of the rows of x over a Q8 lm_head (tsm_lm_head_q8): wq int8
    [vocab, dim], wscale the f16 block scales as int16/uint16 bit patterns
    [vocab, dim / 32]; the rows are normalized and quantized per 32-value
    block as the reference does, and the integer block dots run on the int8
    MFMA cores."""
    import torch

    if x.dtype != torch.float32 or norm_w.dtype != torch.float32 or wq.dtype != torch.int8 or \
            wscale.dtype not in (torch.int16, torch.uint16):
        raise TypeError("x and norm_w must be float32, wq int8, wscale 16-bit")
    if not (x.is_cuda and norm_w.is_cuda and wq.is_cuda and wscale.is_cuda):
        raise ValueError("x, norm_w, wq and wscale must be on the GPU")
    if x.dim() != 2 or x.stride(1) != 1 or not wq.is_contiguous() or not wscale.is_contiguous():
        raise ValueError("x must be [rows, dim] with unit column stride; wq and wscale contiguous")
    rows, dim = x.shape
    vocab = wq.shape[0]
    if wq.shape[1] != dim or wscale.shape != (vocab, dim // 32) or norm_w.numel() != dim:
        raise ValueError("shapes disagree")
    need = workspace_bytes_q8(rows, dim)
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    if out is None:
        out = torch.empty(rows, vocab, dtype=torch.float32, device=x.device)
    err = _lib._err()
    s = stream if stream is not None else torch.cuda.current_stream().cuda_stream
    rc = _lib.lib().tsm_lm_head_q8(s, x.data_ptr(), x.stride(0), norm_w.data_ptr(), float(eps), wq.data_ptr(),
                                   wscale.data_ptr(), rows, dim, vocab, workspace.data_ptr(),
                                   workspace.numel() * workspace.element_size(), out.data_ptr(), out.stride(0),
                                   err, len(err))
    if rc != 0:
        raise _lib.TsmError(err.value.decode())
    return out
