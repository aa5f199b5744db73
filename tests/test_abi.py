"""CPU checks of the C-ABI boundary: the library loads, exports every entry
point include/flaxchat_amd.h declares, its structures match the ctypes
mirror byte for byte, and argument errors come back as status codes
(no GPU call is made)."""

import ctypes
import os
import re
import subprocess

import pytest

from flaxchat_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "flaxchat_amd.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(fc_\w+)\s*\(", src)))


def test_library_loads_and_exports_every_declared_symbol():
    L = _lib.lib()
    names = declared_functions()
    assert len(names) >= 15
    for n in names:
        assert hasattr(L, n), f"{n} declared in the header but not exported"
    assert set(_lib.EXPORTS) == set(names)


def test_version_and_error_string():
    L = _lib.lib()
    assert L.fc_version() >= 100
    assert isinstance(L.fc_last_error(), bytes)


def test_argument_errors_are_status_codes():
    L = _lib.lib()
    rc = L.fc_gemm(None, None, None, 1, 1, 8, 0, 0, None)
    assert rc == -1 and b"null" in L.fc_last_error()
    rc = L.fc_attention(None, None, None, None, 1, 1, 1, 1, 1, 128, 32, None, None, 0, 1, 1, None, 0, None)
    assert rc == -1
    rc = L.fc_attention_noalloc(None, None, None, None, 1, 1, 1, 1, 1, 128, 32, None, None, 0, 1, 1, None)
    assert rc == -1 and b"null" in L.fc_last_error()
    assert L.fc_attention_noalloc_max_bytes() == 32 << 20
    st = _lib.FcSpecState()
    assert L.fc_spec_accept(ctypes.byref(st), None) == -1
    m, c = _lib.FcModel(), _lib.FcCache()
    assert L.fc_attn_prologue(ctypes.byref(m), 0, ctypes.byref(c), None, None, None, None, None, 1, None, None) == -1
    assert b"null" in L.fc_last_error()
    assert L.fc_attn_qkv(ctypes.byref(m), 0, ctypes.byref(c), None, None, None, None, 1, 0, None, None, 0, None) == -1
    # the measurement probes refuse null pointers and bad sizes before any GPU call
    p = ctypes.c_void_p(0x1000)
    assert L.fc_read_probe(None, 4096, p, 1, None) == -1 and b"null" in L.fc_last_error()
    assert L.fc_read_probe(p, 4100, p, 1, None) == -1
    assert L.fc_read_probe(p, 4096, p, 0, None) == -1
    assert L.fc_l2_read_probe(p, 1000, 1 << 20, p, 8, None) == -1
    assert L.fc_l2_read_probe(p, 65536, 1 << 10, p, 8, None) == -1  # under 64 KB per workgroup
    assert L.fc_walk_probe(None, 4, 2, p, None) == -1 and b"null" in L.fc_last_error()
    assert L.fc_walk_probe(p, 0, 2, p, None) == -1
    assert L.fc_walk_probe(p, 4, 0, p, None) == -1
    assert L.fc_gemm_walk_probe(None, p, 32, 64, 256, 32, 32, 1, 0, p, None) == -1 and b"null" in L.fc_last_error()
    assert L.fc_gemm_walk_probe(p, p, 32, 64, 288, 32, 32, 1, 0, p, None) == -1  # K not a multiple of 64
    assert L.fc_gemm_walk_probe(p, p, 32, 64, 256, 32, 48, 1, 0, p, None) == -1  # tile_n does not divide N
    assert L.fc_gemm_walk_probe(p, p, 32, 64, 256, 24, 32, 1, 0, p, None) == -1  # tile_m not a multiple of 16
    assert L.fc_gemm_walk_probe(p, p, 32, 64, 256, 32, 32, 5, 0, p, None) == -1  # more splits than 64-deep chunks
    assert L.fc_gemm_walk_probe_words(224, 4608, 32, 128, 1) == 4 * 8 * 32  # 252 tiles -> 8 x 32 workgroups
    assert L.fc_gemm_walk_probe_words(0, 64, 32, 32, 1) == -1


def test_noalloc_refuses_sizes_beyond_scratch():
    """Sizes whose split-KV partials exceed the static scratch are refused
    with FC_ERR_CAPACITY before any HIP call, so non-null dummy addresses are
    never dereferenced (and a regression returns an error here instead of
    launching over them on a GPU)."""
    L = _lib.lib()
    cap_bytes = L.fc_attention_noalloc_max_bytes()
    assert cap_bytes > 0
    # 4096 rows x 16 KV groups x 64-token chunks (64 query columns per group:
    # the split decode kernel, not the prefill one) need far more partials
    need = L.fc_attention_workspace_bytes(4096, 64, 16, 16, 128, 8192)
    assert need > cap_bytes
    p = 0x1000
    rc = L.fc_attention_noalloc(p, p, p, p, 4096, 4096 * 64, 64, 16, 16, 128, 8192, p, p, 0, 8192, _lib.FC_BF16,
                                None)
    assert rc == -4 and b"scratch" in L.fc_last_error()


def test_struct_layout_matches_c(tmp_path):
    """Compile a C probe against the header and compare sizes and offsets."""
    fields = {
        "fc_layer": _lib.FcLayer, "fc_model": _lib.FcModel, "fc_cache": _lib.FcCache,
        "fc_chunk": _lib.FcChunk, "fc_rowstat": _lib.FcRowstat, "fc_spec_state": _lib.FcSpecState,
    }
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void){"]
    for cname, cls in fields.items():
        lines.append(f'printf("{cname} %zu\\n", sizeof({cname}));')
        for fname, _ in cls._fields_:
            lines.append(f'printf("{cname}.{fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("return 0;}")
    c = tmp_path / "probe.c"
    c.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", str(c), "-o", str(exe)], check=True)
    out = dict(l.rsplit(" ", 1) for l in subprocess.run([str(exe)], capture_output=True, text=True,
                                                         check=True).stdout.split("\n") if l)
    for cname, cls in fields.items():
        assert int(out[cname]) == ctypes.sizeof(cls), cname
        for fname, _ in cls._fields_:
            assert int(out[f"{cname}.{fname}"]) == getattr(cls, fname).offset, f"{cname}.{fname}"


def test_workspace_size_query_needs_no_gpu():
    from flaxchat_amd.config import GPTConfig
    m = _lib.FcModel()
    m.n_layer, m.n_embd, m.n_head, m.n_kv_head, m.head_dim = 2, 256, 2, 2, 128
    m.vocab = m.vocab_pad = 8192
    m.dtype = 1
    nb = _lib.lib().fc_forward_workspace_bytes(ctypes.byref(m), 4, 20, 5, 0)
    assert nb > 20 * 256 * 4 * 3
    assert _lib.lib().fc_attention_workspace_bytes(4, 5, 6, 6, 128, 1024) > 0


def test_workspace_sizing_for_narrow_fp32_models():
    """Workspace sizing is host arithmetic only. An fp32 model narrower than a
    64-column GEMM tile (n_embd 32) once divided by zero while planning bf16
    K splits the fp32 path never uses; it must return a size."""
    L = _lib.lib()
    layers = (_lib.FcLayer * 2)()
    lp = ctypes.cast(layers, ctypes.POINTER(_lib.FcLayer))
    tgt = _lib.FcModel(2, 32, 2, 1, 16, 128, 128, _lib.FC_F32, 1, 1, 1, 0.0, 0.2, 1, 1, 640, lp)
    drf = _lib.FcModel(1, 32, 2, 1, 16, 128, 128, _lib.FC_F32, 1, 1, 1, 0.0, 0.2, 1, 1, 640, lp)
    assert L.fc_spec_workspace_bytes(ctypes.byref(tgt), ctypes.byref(drf), 1, 3) > 0
    for M in (1, 5, 16, 40):
        assert L.fc_forward_workspace_bytes(ctypes.byref(tgt), 1, M, M, M) > 0
