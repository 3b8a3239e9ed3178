"""The C ABI: the library loads without a GPU, exports every function that
include/bolt3_amd.h declares, and the ctypes mirrors of the argument structs
have the C layout (field offsets and sizes taken from gcc on the header)."""
import ctypes
import os
import re
import subprocess
import tempfile

import pytest

from bolt3_amd import _abi as A

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "bolt3_amd.h")


def _declared_functions():
    txt = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|int32_t|int64_t|const char\s*\*)\s*(bolt3_\w+)\s*\(", txt, re.M)))


def test_header_declares_the_bound_functions():
    assert _declared_functions() == sorted(A.EXPORTS)


def test_library_loads_and_exports_everything():
    if not os.path.exists(A.LIB_PATH):
        pytest.fail("libbolt3_amd.so not built (run __graft_entry__.build())")
    lib = A.load()
    for name in _declared_functions():
        assert hasattr(lib, name), name
    assert b"gfx950" in lib.bolt3_version()


def test_workspace_size_formula():
    lib = A.load()
    # per (step, bh): w, bsafe and 1/|k| rows of 256 floats; fp32 / HD=128 adds the roped slot keys per bh
    rows = lambda steps, bh: 3 * steps * bh * 256 * 4
    assert lib.bolt3_chain_workspace_bytes(1, 4, 8, 128, 128, 30) == rows(30, 32)
    assert lib.bolt3_chain_workspace_bytes(0, 1, 3, 64, 128, 1) == rows(1, 3)
    assert lib.bolt3_chain_workspace_bytes(0, 2, 2, 128, 128, 5) == rows(5, 4) + 4 * 128 * 128 * 4


def test_rejects_bad_arguments_without_gpu_work():
    """Argument checks run on the host before any launch."""
    lib = A.load()
    a = A.ChainArgs()
    a.B, a.HKV, a.HD, a.S, a.n_steps = 1, 1, 96, 128, 1
    assert lib.bolt3_chain(ctypes.byref(a), None) == 1002      # unsupported head dim
    a.HD, a.S = 128, 64
    assert lib.bolt3_chain(ctypes.byref(a), None) == 1002      # unsupported slot count
    a.S, a.len0 = 128, 300
    assert lib.bolt3_chain(ctypes.byref(a), None) == 1002      # chunk longer than 256 tokens
    a.len0 = 128
    assert lib.bolt3_chain(ctypes.byref(a), None) == 1001      # null pointers
    h = A.HeadsArgs()
    assert lib.bolt3_heads(ctypes.byref(h), None) == 1001
    t = A.AttnArgs()
    assert lib.bolt3_chunk_attn(ctypes.byref(t), None) == 1001
    d = A.DecodeArgs()
    assert lib.bolt3_decode(ctypes.byref(d), None) == 1001
    la = A.DecodeLayerArgs()
    la.dec.dtype = 0
    assert lib.bolt3_decode_layer(ctypes.byref(la), None) == 1002   # fp32: the unfused step only
    la.dec.dtype = 1
    assert lib.bolt3_decode_layer(ctypes.byref(la), None) == 1001
    assert lib.bolt3_wait_count(None, 1, 10, None) == 1001
    assert lib.bolt3_chain_noalloc(None, None) == 1001
    big = A.ChainArgs()
    big.dtype, big.B, big.HKV, big.HD, big.S, big.n_steps = 1, 64, 8, 128, 128, 100
    assert lib.bolt3_chain_noalloc(ctypes.byref(big), None) == 1003   # beyond the library's scratch
    sk = A.SlotKeysArgs()
    sk.dtype, sk.B, sk.HKV, sk.HD, sk.S = 1, 1, 1, 128, 128
    assert lib.bolt3_slot_keys(ctypes.byref(sk), None) == 1001        # null pointers
    sk.S = 64
    assert lib.bolt3_slot_keys(ctypes.byref(sk), None) == 1002        # S != 128
    cb = A.ChainBwdArgs()
    cb.dtype, cb.B, cb.HKV, cb.HD, cb.S, cb.T = 2, 1, 1, 128, 128, 512
    cb.n_steps, cb.off0, cb.len0, cb.step_stride, cb.step_len = 2, 4, 124, 128, 128
    assert lib.bolt3_chain_bwd(ctypes.byref(cb), None) == 1002        # unknown dtype code
    cb.dtype, cb.HD = 1, 96
    assert lib.bolt3_chain_bwd(ctypes.byref(cb), None) == 1002        # head dim not 64 or 128
    cb.HD, cb.S = 64, 64
    assert lib.bolt3_chain_bwd(ctypes.byref(cb), None) == 1002        # S != 128
    cb.S = 128
    for dt, hd in ((0, 64), (0, 128), (1, 64)):                       # fp32 and head dim 64 are taken
        cb.dtype, cb.HD = dt, hd
        assert lib.bolt3_chain_bwd(ctypes.byref(cb), None) == 1001    # (null pointers)
    cb.dtype, cb.HD, cb.step_len = 1, 128, 200
    assert lib.bolt3_chain_bwd(ctypes.byref(cb), None) == 1002        # steps longer than 128 tokens
    cb.step_len, cb.T = 128, 200
    assert lib.bolt3_chain_bwd(ctypes.byref(cb), None) == 1001        # steps past the sequence
    cb.T = 512
    assert lib.bolt3_chain_bwd(ctypes.byref(cb), None) == 1001        # null pointers
    assert lib.bolt3_chain_bwd_workspace_bytes(4, 8, 128, 30) == 4 * 30 * 32 * 4 * 128 + 30 * 32 * 128 * 128 * 4
    assert lib.bolt3_chain_bwd_workspace_bytes(4, 8, 64, 30) == 4 * 30 * 32 * 4 * 128 + 30 * 32 * 64 * 64 * 4
    assert lib.bolt3_chain_bwd_workspace_bytes(4, 8, 96, 30) == 0
    d2 = A.DecodeArgs()
    d2.dtype, d2.B, d2.H, d2.HKV, d2.HD, d2.S, d2.has_slots = 1, 1, 4, 1, 128, 256, 1
    assert lib.bolt3_decode(ctypes.byref(d2), None) in (1001, 1002)   # rejected before any launch


STRUCTS = {"b3_heads_args": A.HeadsArgs, "b3_chain_args": A.ChainArgs, "b3_attn_args": A.AttnArgs,
           "b3_decode_args": A.DecodeArgs, "b3_decode_layer_args": A.DecodeLayerArgs,
           "b3_slot_keys_args": A.SlotKeysArgs, "b3_attn_bwd_args": A.AttnBwdArgs,
           "b3_rms_norm_args": A.RmsNormArgs, "b3_chain_bwd_args": A.ChainBwdArgs,
           "b3_heads_bwd_args": A.HeadsBwdArgs}


def _flat_fields(st, prefix=""):
    for name, typ in st._fields_:
        yield prefix + name, getattr(st, name).offset, ctypes.sizeof(typ)


def test_struct_layout_matches_header():
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void) {"]
    for cname, st in STRUCTS.items():
        lines.append(f'printf("{cname} sizeof %zu\\n", sizeof({cname}));')
        for field, _, _ in _flat_fields(st):
            lines.append(f'printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines.append("return 0; }")
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "probe.c"), os.path.join(d, "probe")
        open(src, "w").write("\n".join(lines))
        subprocess.run(["gcc", "-std=c99", src, "-o", exe], check=True)
        out = subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split("\n")
    got = {}
    for ln in out:
        if ln:
            s, f, v = ln.split()
            got[(s, f)] = int(v)
    for cname, st in STRUCTS.items():
        assert got[(cname, "sizeof")] == ctypes.sizeof(st), cname
        for field, off, _ in _flat_fields(st):
            assert got[(cname, field)] == off, (cname, field)


def test_no_packed_fp32_in_device_code():
    """The build keeps packed fp32 VALU ops out of the code objects (-Xclang -target-feature
    -Xclang -packed-fp32-ops acts on the device pass; only the host pass warns that it does not
    know it): every kernel source compiled to gfx950 assembly has none."""
    import re
    from bolt3_amd import build as Bd
    pat = re.compile(r"\bv_pk_(" + "|".join(("add", "mul", "fma")) + r")_f32\b")
    with tempfile.TemporaryDirectory() as d:
        for src in Bd.sources():
            out = os.path.join(d, os.path.basename(src) + ".s")
            r = subprocess.run([Bd.HIPCC, *Bd.FLAGS, "-S", "--cuda-device-only", src, "-o", out],
                               capture_output=True, text=True)
            assert r.returncode == 0, r.stderr[-2000:]
            assert not pat.search(open(out).read()), src


def test_noalloc_scratch_size_matches_header():
    txt = open(HEADER).read()
    m = re.search(r"#define B3_CHAIN_NOALLOC_SCRATCH_BYTES \((\d+) << (\d+)\)", txt)
    assert m and int(m.group(1)) << int(m.group(2)) == A.CHAIN_NOALLOC_SCRATCH_BYTES



def test_chain_bwd_kernel_bits_match_header():
    txt = open(HEADER).read()
    bits = {k: int(v) for k, v in re.findall(r"#define B3_CBWD_(\w+) (\d+)", txt)}
    assert bits == {"STATS": A.CBWD_STATS, "M_REC": A.CBWD_M_REC, "SLOT_REC": A.CBWD_SLOT_REC,
                    "TOK_GRAD": A.CBWD_TOK_GRAD, "ALL": 15}
    # a mask outside the four bits is rejected before any launch
    lib = A.load()
    cb = A.ChainBwdArgs()
    cb.dtype, cb.B, cb.HKV, cb.HD, cb.S, cb.T = 1, 1, 1, 128, 128, 512
    cb.n_steps, cb.off0, cb.len0, cb.step_stride, cb.step_len = 2, 4, 124, 128, 128
    cb.kernels = 16
    assert lib.bolt3_chain_bwd(ctypes.byref(cb), None) == 1001
