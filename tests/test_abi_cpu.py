"""The C ABI without a GPU: the library builds, loads and exports every
function include/tachyon_sampler.h declares; the struct layouts seen by a C
compiler match the ctypes mirror; argument errors come back as messages."""
import ctypes
import os
import re
import subprocess

import pytest

from tachyon_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tachyon_sampler.h")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:[\w\*]+\s+)+\**(tsm_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    names = declared_functions()
    assert set(names) == set(_lib.SYMBOLS), names
    for name in names:
        assert hasattr(L, name), name
    assert L.tsm_version().decode().startswith("tachyon-sampler")


def test_static_archive_has_the_symbols():
    a = os.path.join(ROOT, "tachyon_amd", "lib", "libtachyon_sampler.a")
    out = subprocess.run(["nm", "-g", "--defined-only", a], capture_output=True, text=True, check=True).stdout
    for name in declared_functions():
        assert re.search(rf"\bT {name}\b", out), name


def test_struct_layout_matches_c(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text(f'''
#include <stdio.h>
#include <stddef.h>
#include "{HEADER}"
int main(void) {{
  printf("%zu %zu %zu\\n", sizeof(tsm_row_params), sizeof(tsm_batch), sizeof(tsm_outputs));
  printf("%zu %zu %zu %zu\\n", offsetof(tsm_batch, params), offsetof(tsm_batch, uniforms),
         offsetof(tsm_outputs, top_stride), offsetof(tsm_outputs, keep));
  printf("%zu %zu %zu %zu\\n", sizeof(tsm_json_state), offsetof(tsm_json_state, whitespace),
         sizeof(tsm_vocab), offsetof(tsm_vocab, n_tokens));
  return 0;
}}''')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", str(src), "-o", str(exe)], check=True)
    l1, l2, l3 = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n")[:3]
    from tachyon_amd.workloads import ROW_PARAMS_DTYPE

    assert [int(v) for v in l1.split()] == [ROW_PARAMS_DTYPE.itemsize, ctypes.sizeof(_lib.TsmBatch),
                                            ctypes.sizeof(_lib.TsmOutputs)]
    assert [int(v) for v in l2.split()] == [_lib.TsmBatch.params.offset, _lib.TsmBatch.uniforms.offset,
                                            _lib.TsmOutputs.top_stride.offset, _lib.TsmOutputs.keep.offset]
    assert [int(v) for v in l3.split()] == [ctypes.sizeof(_lib.TsmJsonState), _lib.TsmJsonState.whitespace.offset,
                                            ctypes.sizeof(_lib.TsmVocab), _lib.TsmVocab.n_tokens.offset]


def _no_gpu():
    try:
        import torch

        return not torch.cuda.is_available()
    except Exception:
        return True


@pytest.mark.skipif(not _no_gpu(), reason="checks the no-device error path")
def test_create_without_a_device_reports_an_error():
    L = _lib.lib()
    err = ctypes.create_string_buffer(256)
    h = L.tsm_create(0, 16, 1000, err, len(err))
    assert not h
    assert err.value  # a message, not a crash


def test_argument_errors_need_no_device():
    L = _lib.lib()
    err = ctypes.create_string_buffer(256)
    assert not L.tsm_create(0, 0, 1000, err, len(err))
    assert b"max_rows" in err.value
    assert not L.tsm_create(0, 16, 0, err, len(err))
    assert b"max_vocab" in err.value
    assert L.tsm_sample(None, None, None, None, err, len(err)) != 0
    assert L.tsm_distribution(None, None, None, None, None, 0, None, err, len(err)) != 0
    assert L.tsm_status(None, None, err, len(err)) != 0
    L.tsm_destroy(None)
    # the mask producer checks its arguments on the host before any launch
    assert L.tsm_json_mask(None, None, None, 1, 10, None, 1, err, len(err)) != 0
    assert b"vocab" in err.value
    v = _lib.TsmVocab(None, None, None, 0, 0)
    st = _lib.TsmJsonState()
    assert L.tsm_json_mask(None, ctypes.byref(v), ctypes.byref(st), 1, 100, ctypes.byref(st), 1, err, len(err)) != 0
    assert b"mask_stride" in err.value


def test_lm_head_arguments_are_checked_on_the_host():
    L = _lib.lib()
    err = ctypes.create_string_buffer(256)
    # workspace: the bf16 operands of the rows padded to the workgroup tile
    # (16, 32, 64, 128 or 256 rows), twice when split
    assert L.tsm_lm_head_workspace(1, 4096, 0) == 16 * 4096 * 2
    assert L.tsm_lm_head_workspace(17, 4096, 0) == 32 * 4096 * 2
    assert L.tsm_lm_head_workspace(33, 4096, 0) == 64 * 4096 * 2
    assert L.tsm_lm_head_workspace(100, 4096, 0) == 128 * 4096 * 2
    assert L.tsm_lm_head_workspace(256, 4096, 0) == 256 * 4096 * 2
    assert L.tsm_lm_head_workspace(257, 4096, _lib.LM_SPLIT) == 512 * 4096 * 2 * 2
    fake = ctypes.c_void_p(0x10000)  # never dereferenced: every case below fails its checks first
    def call(rows=4, dim=128, vocab=100, flags=0, ws=1 << 20, ld=100, x_stride=128, w=fake):
        return L.tsm_lm_head(None, fake, x_stride, fake, 1e-5, w, rows, dim, vocab, flags, fake, ws, fake, ld,
                             err, len(err))
    assert call(dim=100) != 0 and b"multiple of 64" in err.value
    assert call(rows=0) != 0 and b"rows" in err.value
    assert call(vocab=0) != 0 and b"vocab" in err.value
    assert call(ld=99) != 0 and b"ld" in err.value
    assert call(x_stride=64) != 0 and b"x_stride" in err.value
    assert call(flags=4) != 0 and b"flags" in err.value
    assert call(ws=1000) != 0 and b"workspace" in err.value
    assert call(w=ctypes.c_void_p(0x10008)) != 0 and b"aligned" in err.value


def test_lm_head_q8_arguments_are_checked_on_the_host():
    L = _lib.lib()
    err = ctypes.create_string_buffer(256)
    # workspace: the activation fragments (1 KB per 16 padded rows and pair
    # of 32-value blocks), then one f32 scale per padded row and block
    assert L.tsm_lm_head_q8_workspace(1, 4096) == 1 * 64 * 1024 + 16 * 128 * 4
    assert L.tsm_lm_head_q8_workspace(17, 96) == 2 * 2 * 1024 + 32 * 3 * 4
    assert L.tsm_lm_head_q8_workspace(3, 32) == 1 * 1 * 1024 + 16 * 1 * 4
    fake = ctypes.c_void_p(0x10000)  # never dereferenced: every case below fails its checks first
    def call(rows=4, dim=128, vocab=100, ws=1 << 20, ld=100, x_stride=128, w=fake, s=fake):
        return L.tsm_lm_head_q8(None, fake, x_stride, fake, 1e-5, w, s, rows, dim, vocab, fake, ws, fake, ld,
                                err, len(err))
    assert call(dim=100) != 0 and b"multiple of 32" in err.value
    assert call(rows=0) != 0 and b"rows" in err.value
    assert call(vocab=0) != 0 and b"vocab" in err.value
    assert call(ld=99) != 0 and b"ld" in err.value
    assert call(x_stride=64) != 0 and b"x_stride" in err.value
    assert call(ws=1000) != 0 and b"workspace" in err.value
    assert call(w=ctypes.c_void_p(0x10008)) != 0 and b"aligned" in err.value
    assert call(s=ctypes.c_void_p(0x10001)) != 0 and b"aligned" in err.value
    assert call(w=None) != 0 and b"must be set" in err.value


def test_lm_head_q8_wrapper_checks_its_arguments_before_any_gpu_call():
    """tachyon_amd.lmhead.lm_head_q8 rejects wrong dtypes, host tensors and
    shapes that disagree before it queues anything (so this runs without a
    GPU)."""
    import torch

    from tachyon_amd.lmhead import lm_head_q8

    x = torch.zeros(2, 64)
    g = torch.ones(64)
    wq = torch.zeros(10, 64, dtype=torch.int8)
    ws = torch.zeros(10, 2, dtype=torch.int16)
    with pytest.raises(TypeError):
        lm_head_q8(x.double(), g, 1e-5, wq, ws)
    with pytest.raises(TypeError):
        lm_head_q8(x, g, 1e-5, wq.to(torch.uint8), ws)
    with pytest.raises(TypeError):
        lm_head_q8(x, g, 1e-5, wq, ws.float())
    with pytest.raises(ValueError, match="GPU"):
        lm_head_q8(x, g, 1e-5, wq, ws)
