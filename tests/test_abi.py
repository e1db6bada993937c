"""The C ABI of libmuzero_hip.so (CPU checks; no kernel is launched).

* every entry point declared in include/muzero_hip.h is exported and has a
  ctypes signature in muzero_amd/_lib.py;
* the ctypes mirror of ``mz_decode_args`` has exactly the field offsets and
  size that a C compiler gives the header's struct;
* argument validation that happens before any device work (status codes,
  error strings) behaves as documented.
"""

import ctypes
import os
import re
import shutil
import subprocess

import pytest

from muzero_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "muzero_hip.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(muzero_[a-z_0-9]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = _declared_functions()
    for required in ("muzero_quantize_rows", "muzero_quantize_keys", "muzero_quantize_values",
                     "muzero_dequantize_rows", "muzero_decode_attention", "muzero_decode_workspace_bytes"):
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared_functions():
        assert hasattr(lib, name), f"{name} declared in the header but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"


def test_version_and_strerror():
    lib = _lib.load()
    assert lib.muzero_version().decode().startswith("muzero_hip")
    for code in (0, -1, -2, -3, -4):
        assert lib.muzero_strerror(code)


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
@pytest.mark.parametrize("cls,cname", [(_lib.DecodeArgs, "mz_decode_args"), (_lib.PrologueArgs, "mz_prologue_args"),
                                       (_lib.QkArgs, "mz_qk_args"), (_lib.AvArgs, "mz_av_args"),
                                       (_lib.PrefixStateArgs, "mz_prefix_state_args")])
def test_args_layout_matches_c(tmp_path, cls, cname):
    fields = [f for f, _ in cls._fields_]
    src = ['#include <stddef.h>', '#include <stdio.h>', f'#include "{HEADER}"', "int main(void) {",
           f'  printf("size %zu\\n", sizeof({cname}));']
    src += [f'  printf("{f} %zu\\n", offsetof({cname}, {f}));' for f in fields]
    src += ["  return 0;", "}"]
    c = tmp_path / "layout.c"
    c.write_text("\n".join(src))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-o", str(exe), str(c)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    got = dict(line.split() for line in out if line)
    assert int(got["size"]) == ctypes.sizeof(cls)
    for f in fields:
        assert int(got[f]) == getattr(cls, f).offset, f


def test_decode_workspace_rejects_bad_args_without_a_device():
    """Host-side validation: unsupported head_dim / n_rep / bits are rejected (-1) before any launch."""
    lib = _lib.load()
    a = _lib.DecodeArgs()
    a.batch, a.kv_heads, a.n_rep, a.head_dim, a.bits = 1, 1, 4, 96, 4
    a.n_groups, a.n_residual = 0, 16
    assert lib.muzero_decode_workspace_bytes(ctypes.byref(a), None) == -1
    a.head_dim, a.bits = 128, 9
    assert lib.muzero_decode_workspace_bytes(ctypes.byref(a), None) == -1


def test_noalloc_rejects_partials_beyond_the_scratch_without_a_device():
    """muzero_decode_attention_noalloc checks the split partials' size against its static scratch
    (MZ_DECODE_SCRATCH_BYTES) on the host and returns MZ_ESCRATCH before any device work: 64 batch
    rows x 8 kv heads x 4 q heads x 64 forced splits x 130 floats is 17 MB.  The pointers are
    placeholders: nothing is read."""
    lib = _lib.load()
    a = _lib.DecodeArgs()
    a.batch, a.kv_heads, a.n_rep, a.head_dim, a.bits = 64, 8, 4, 128, 4
    a.n_groups, a.n_residual, a.n_split = 62, 128, 64
    a.meta_dtype, a.io_dtype, a.out_dtype = _lib.MZ_F16, _lib.MZ_BF16, _lib.MZ_BF16
    fake = 1 << 20
    a.query = a.k_packed = a.k_mn = a.k_scale = a.v_packed = a.v_mn = a.v_scale = fake
    a.k_res = a.v_res = a.e_key = a.e_value = a.out = fake
    a.q_sb, a.q_sh = 32 * 128, 128
    a.kr_sb, a.kr_sh, a.kr_st = 8 * 128 * 128, 128 * 128, 128
    a.vr_sb, a.vr_sh, a.vr_st = a.kr_sb, a.kr_sh, a.kr_st
    ns = ctypes.c_int(0)
    need = lib.muzero_decode_workspace_bytes(ctypes.byref(a), ctypes.byref(ns))
    assert ns.value == 64 and need == 64 * 32 * 64 * 130 * 4 > _lib.MZ_DECODE_SCRATCH_BYTES
    assert lib.muzero_decode_attention_noalloc(ctypes.byref(a), None) == _lib.MZ_ESCRATCH
    assert b"scratch" in lib.muzero_strerror(_lib.MZ_ESCRATCH)


def test_qk_av_reject_bad_args_without_a_device():
    """muzero_qk / muzero_av validate on the host: bad bits, n_rep and head_dim are rejected
    before any launch, and an empty call returns 0 without touching a device."""
    lib = _lib.load()
    a = _lib.QkArgs()
    a.batch, a.kv_heads, a.n_rep, a.head_dim, a.bits, a.n_groups = 1, 1, 4, 128, 9, 1
    assert lib.muzero_qk(ctypes.byref(a), None) == -1
    a.bits, a.n_rep = 4, 17
    assert lib.muzero_qk(ctypes.byref(a), None) == -2
    a.n_rep, a.head_dim = 4, 512
    assert lib.muzero_qk(ctypes.byref(a), None) == -2
    a.head_dim, a.n_groups = 128, 0
    assert lib.muzero_qk(ctypes.byref(a), None) == 0
    a.n_groups = 1  # null pointers with work to do
    assert lib.muzero_qk(ctypes.byref(a), None) == -1
    v = _lib.AvArgs()
    v.batch, v.kv_heads, v.n_rep, v.head_dim, v.bits, v.n_tokens = 1, 1, 4, 128, 0, 5
    assert lib.muzero_av(ctypes.byref(v), None) == -1
    v.bits, v.head_dim = 4, 300
    assert lib.muzero_av(ctypes.byref(v), None) == -2
    v.head_dim, v.batch = 128, 0
    assert lib.muzero_av(ctypes.byref(v), None) == 0


def test_stream_read_rejects_bad_args_without_a_device():
    """muzero_stream_read checks pointers, alignment, size and the output count on the host."""
    lib = _lib.load()
    src, out = ctypes.c_void_p(4096), ctypes.c_void_p(8192)
    assert lib.muzero_stream_read(None, 16, out, 1, None) == -1
    assert lib.muzero_stream_read(src, 16, None, 1, None) == -1
    assert lib.muzero_stream_read(src, 15, out, 1, None) == -1
    assert lib.muzero_stream_read(ctypes.c_void_p(4100), 16, out, 1, None) == -1
    assert lib.muzero_stream_read(src, 16, out, 0, None) == -1
    assert lib.muzero_stream_read(src, 16, out, 65536, None) == -1
    assert lib.muzero_stream_read(src, -16, out, 1, None) == -1


def test_noalloc_status_codes_match_the_workspace_entry_point_without_a_device():
    """muzero_decode_attention_noalloc returns the status muzero_decode_attention gives for the same
    arguments when the arguments are rejected: MZ_EUNSUPPORTED for head_dim 96 and for n_rep 17,
    MZ_EINVAL for bits 9 (all before any device work; the pointers are placeholders)."""
    lib = _lib.load()
    a = _lib.DecodeArgs()
    a.batch, a.kv_heads, a.n_rep, a.head_dim, a.bits = 1, 1, 4, 96, 4
    a.n_groups, a.n_residual = 0, 16
    a.meta_dtype, a.io_dtype, a.out_dtype = _lib.MZ_F16, _lib.MZ_BF16, _lib.MZ_BF16
    for field, value, want in (("head_dim", 96, -2), ("n_rep", 17, -2), ("bits", 9, -1)):
        b = _lib.DecodeArgs.from_buffer_copy(a)
        b.head_dim = 128
        setattr(b, field, value)
        assert lib.muzero_decode_attention(ctypes.byref(b), None) == want, field
        assert lib.muzero_decode_attention_noalloc(ctypes.byref(b), None) == want, field


def test_prefix_state_rejects_bad_args_without_a_device():
    """muzero_decode_prefix_state takes the packed prefix alone: a residual, a negative chunk count,
    missing outputs or chunk records are rejected (MZ_EINVAL) before any device work; an empty batch
    is a no-op."""
    lib = _lib.load()
    a = _lib.DecodeArgs()
    a.batch, a.kv_heads, a.n_rep, a.head_dim, a.bits = 1, 1, 4, 128, 4
    a.n_groups, a.n_residual = 2, 0
    a.meta_dtype, a.io_dtype, a.out_dtype = _lib.MZ_F16, _lib.MZ_BF16, _lib.MZ_BF16
    fake = 1 << 20
    a.query = a.k_packed = a.k_mn = a.k_scale = a.v_packed = a.v_mn = a.v_scale = a.e_key = a.e_value = fake
    a.out = fake
    st = _lib.PrefixStateArgs()
    assert lib.muzero_decode_prefix_state(ctypes.byref(a), ctypes.byref(st), None) == -1  # no outputs
    st.acc = st.m = st.l = fake
    st.n_chunks = -1
    assert lib.muzero_decode_prefix_state(ctypes.byref(a), ctypes.byref(st), None) == -1
    st.n_chunks = 3  # chunk records missing
    assert lib.muzero_decode_prefix_state(ctypes.byref(a), ctypes.byref(st), None) == -1
    st.n_chunks = 0
    a.n_residual = 16  # not a prefix-only call
    assert lib.muzero_decode_prefix_state(ctypes.byref(a), ctypes.byref(st), None) == -1
    a.n_residual = 0
    assert lib.muzero_decode_prefix_state(ctypes.byref(a), ctypes.byref(st), None) == -3  # no workspace
    a.head_dim = 96
    assert lib.muzero_decode_prefix_state(ctypes.byref(a), ctypes.byref(st), None) == -2
    a.head_dim, a.batch = 128, 0
    assert lib.muzero_decode_prefix_state(ctypes.byref(a), ctypes.byref(st), None) == 0
