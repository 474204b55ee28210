"""JSON-object constraints on the GPU path: the host-side state of Tachyon's
JsonObject (src/constrain.rs:88-302) and the mask producer.

`JsonConstraint` mirrors the reference's Constraint trait for a JsonObject
(`allows`, `advance`, `is_complete`, constrain.rs:35-42) over the library's
packed state (tsm_json_state).  `json_mask` evaluates `allows` for every token
of the vocabulary, for a batch of rows, with one launch (tsm_json_mask), and
writes the packed allow-bits `tsm_sample` consumes.  Everything goes through
the C ABI of the HIP library; there is no CPU fallback for the mask.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib


class JsonConstraint:
    """Constraint for `response_format: json_object` (constrain.rs:14-33)."""

    def __init__(self):
        self.state = _lib.TsmJsonState()
        _lib.lib().tsm_json_init(ctypes.byref(self.state))

    def allows(self, vocab: "HostVocab", token: int) -> bool:
        """constrain.rs:286-290, on the host (one token)."""
        b = vocab.token_bytes(token)
        if vocab.is_special(token) or not b:
            return False
        return bool(_lib.lib().tsm_json_accepts(ctypes.byref(self.state), b, len(b)))

    def accepts(self, b: bytes) -> bool:
        return bool(_lib.lib().tsm_json_accepts(ctypes.byref(self.state), b, len(b)))

    def advance(self, b: bytes) -> None:
        _lib.lib().tsm_json_advance(ctypes.byref(self.state), b, len(b))

    def is_complete(self) -> bool:
        return bool(_lib.lib().tsm_json_is_complete(ctypes.byref(self.state)))

    def packed(self) -> bytes:
        return bytes(self.state)


@dataclass
class HostVocab:
    """A tokenizer's token bytes (tokenizer.rs:189-195) as CSR arrays."""
    bytes: np.ndarray     # uint8, every token's bytes concatenated
    offsets: np.ndarray   # uint32 [n_tokens + 1]
    special: np.ndarray   # uint32 packed bits [ceil(n_tokens / 32)], or None
    n_tokens: int

    @staticmethod
    def from_tokens(tokens, special_ids=()):
        lens = np.fromiter((len(t) for t in tokens), np.int64, len(tokens))
        offsets = np.zeros(len(tokens) + 1, np.uint32)
        offsets[1:] = np.cumsum(lens)
        data = np.frombuffer(b"".join(tokens), np.uint8).copy() if len(tokens) else np.zeros(0, np.uint8)
        special = np.zeros((len(tokens) + 31) // 32, np.uint32)
        for i in special_ids:
            special[i >> 5] |= np.uint32(1 << (i & 31))
        return HostVocab(data if data.size else np.zeros(1, np.uint8), offsets, special, len(tokens))

    def token_bytes(self, t: int) -> bytes:
        if t >= self.n_tokens:
            return b""
        return self.bytes[self.offsets[t]:self.offsets[t + 1]].tobytes()

    def is_special(self, t: int) -> bool:
        return t < self.n_tokens and bool((int(self.special[t >> 5]) >> (t & 31)) & 1)


class DeviceVocab:
    """HostVocab uploaded to the GPU (torch tensors as device memory)."""

    def __init__(self, v: HostVocab, device="cuda:0"):
        import torch

        self.bytes = torch.from_numpy(v.bytes).to(device)
        self.offsets = torch.from_numpy(v.offsets.view(np.int32)).to(device)
        self.special = torch.from_numpy(v.special.view(np.int32)).to(device)
        self.n_tokens = v.n_tokens

    def abi(self):
        return _lib.TsmVocab(self.bytes.data_ptr(), self.offsets.data_ptr(), self.special.data_ptr(),
                             self.n_tokens, 0)


def json_mask(vocab: DeviceVocab, states_dev, rows: int, usable: int, mask_dev, mask_stride: int, stream=None):
    """tsm_json_mask: allow-bits of `rows` rows (states_dev: a uint8 device
    tensor of rows * 12 bytes, tsm_json_state each) into mask_dev."""
    import torch

    s = stream if stream is not None else torch.cuda.current_stream().cuda_stream
    vb = vocab.abi()
    err = _lib._err()
    rc = _lib.lib().tsm_json_mask(ctypes.c_void_p(s), ctypes.byref(vb), ctypes.c_void_p(states_dev.data_ptr()),
                                  rows, usable, ctypes.c_void_p(mask_dev.data_ptr()), mask_stride, err, len(err))
    if rc != 0:
        raise _lib.TsmError(err.value.decode())


class JsonMaskSet:
    """tsm_json_masks_*: masks of recent JsonObject states kept on the GPU;
    each fill evaluates every distinct state of its rows once (reusing the
    kept ones) and copies each row's mask from its state's."""

    def __init__(self, max_rows: int, capacity: int, usable: int, device: int = 0):
        err = _lib._err()
        self.handle = _lib.lib().tsm_json_masks_create(device, max_rows, capacity, usable, err, len(err))
        if not self.handle:
            raise _lib.TsmError(err.value.decode())
        self.usable = usable

    def fill(self, vocab: DeviceVocab, states, mask_dev, mask_stride: int, stream=None):
        """Masks of the rows whose host states are `states` (a sequence of
        JsonConstraint or of packed 12-byte states, or an array from pack())
        into mask_dev; returns the call's counts (rows, distinct, hits,
        evaluated)."""
        import torch

        arr = states if isinstance(states, ctypes.Array) else self.pack(states)
        s = stream if stream is not None else torch.cuda.current_stream().cuda_stream
        vb = vocab.abi()
        st = _lib.TsmJsonFillStats()
        err = _lib._err()
        rc = _lib.lib().tsm_json_masks_fill(self.handle, ctypes.c_void_p(s), ctypes.byref(vb), arr, len(arr),
                                            ctypes.c_void_p(mask_dev.data_ptr()), mask_stride, ctypes.byref(st),
                                            err, len(err))
        if rc != 0:
            raise _lib.TsmError(err.value.decode())
        return (st.rows, st.distinct, st.hits, st.evaluated)

    @staticmethod
    def pack(states):
        """The host array fill() takes: JsonConstraint or packed 12-byte states."""
        packed = [c.packed() if isinstance(c, JsonConstraint) else bytes(c) for c in states]
        arr = (_lib.TsmJsonState * len(packed))()
        ctypes.memmove(arr, b"".join(packed), 12 * len(packed))
        return arr

    def reset(self):
        _lib.lib().tsm_json_masks_reset(self.handle)

    def close(self):
        if self.handle:
            _lib.lib().tsm_json_masks_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def pack_states(constraints) -> np.ndarray:
    """The rows' packed states, ready to upload (uint8, 12 bytes per row)."""
    return np.frombuffer(b"".join(c.packed() for c in constraints), np.uint8).copy()
