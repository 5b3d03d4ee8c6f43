"""CPU-side checks of the C ABI: the library loads, exports every entry point
the public headers declare, validates arguments before touching the GPU, and
its layout math matches the reference constants.  No kernel is launched."""
import ctypes
import os
import re

import numpy as np
import pytest

import fmoe_amd
from fmoe_amd import synth
from fmoe_amd.layout import expert_offsets

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for h in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if not h.endswith(".h"):
            continue
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?[\w]+\s*\*?\s*(fm_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol():
    L = fmoe_amd.lib()
    names = declared_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    # and the Python binding covers them
    assert names <= set(fmoe_amd.SIGNATURES), names - set(fmoe_amd.SIGNATURES)


def test_version_and_error_string():
    L = fmoe_amd.lib()
    assert b"gfx950" in L.fm_version()
    assert isinstance(L.fm_last_error(), bytes)


def test_layout_matches_reference_constants():
    L = fmoe_amd.layout_of(4096, 1024, 64, 4)
    assert list(L.off) == [0, 2097152, 2228224, 2359296, 4456448, 4587520, 4718592, 6815744, 6946816]
    assert L.size == 7077888
    L2 = fmoe_amd.layout_of(4096, 1024, 64, 2)
    assert L2.size == 3932160
    po, ps = expert_offsets(4096, 1024, 64, 2)
    assert list(L2.off) == list(po.values()) and ps == L2.size
    with pytest.raises(fmoe_amd.FmError):
        fmoe_amd.layout_of(4096, 1024, 64, 3)


def test_expert_from_blob_pointer_arithmetic():
    L = fmoe_amd.layout_of(4096, 1024, 64, 4)
    e = fmoe_amd.ExpertWeights()
    base = 1 << 40
    fmoe_amd.check(fmoe_amd.lib().fm_expert_from_blob(ctypes.c_void_p(base), ctypes.byref(L), ctypes.byref(e)))
    assert e.up_w == base + 2359296 and e.down_b == base + 6946816


def test_argument_validation_without_gpu():
    L = fmoe_amd.lib()
    rc = L.fm_dequant_matvec(None, None, None, None, None, 16, 64, 64, 4, None)
    assert rc == -1 and b"NULL" in L.fm_last_error()
    fake = ctypes.c_void_p(1 << 20)
    rc = L.fm_dequant_matvec(fake, fake, fake, fake, fake, 16, 64, 64, 3, None)
    assert rc == -1 and b"bits" in L.fm_last_error()
    rc = L.fm_dequant_matvec(fake, fake, fake, fake, fake, 16, 64, 32, 4, None)
    assert rc == -4 and b"group_size" in L.fm_last_error()
    rc = L.fm_dequant_matvec(fake, fake, fake, fake, fake, 16, 100, 64, 4, None)
    assert rc == -1
    rc = L.fm_dequant_matvec(fake, fake, fake, fake, fake, 16, 64 * 512, 64, 4, None)
    assert rc == -4 and b"16384" in L.fm_last_error()
    rc = L.fm_route_topk(fake, 1, 512, 65, fake, fake, None)
    assert rc == -1 and b"K=65" in L.fm_last_error()
    # decode: K too large, then a workspace that is too small
    rc = L.fm_moe_decode(17, None, None, None, None, None, 4, 0, 0.0, 4096, 1024, 64, fake, None, fake, None,
                         None, 0, None)
    assert rc == -1
    experts = (fmoe_amd.ExpertWeights * 1)()
    for f, _ in fmoe_amd.ExpertWeights._fields_:
        setattr(experts[0], f, 1 << 20)
    bits = (ctypes.c_int * 1)(4)
    w = (ctypes.c_float * 1)(1.0)
    rc = L.fm_moe_decode(1, experts, bits, w, None, None, 4, 0, 0.0, 4096, 1024, 64, fake, None, fake, None, fake,
                         16, None)
    assert rc == -2 and b"workspace" in L.fm_last_error()
    need = L.fm_moe_decode_workspace_size(11, 4096, 1024)
    assert need >= 11 * 1024 * 4


def test_synth_distributions_and_determinism():
    a = synth.expert_blob((1, 2), 4096, 1024, 4)
    b = synth.expert_blob((1, 2), 4096, 1024, 4)
    assert np.array_equal(a, b) and a.size == 7077888
    off, _ = expert_offsets(4096, 1024, 64, 4)
    s = synth.bf16_to_f32(a[off["gate_s"]: off["gate_b"]].view(np.uint16))
    bb = synth.bf16_to_f32(a[off["gate_b"]: off["up_w"]].view(np.uint16))
    assert abs(s.mean() - 0.02 * np.sqrt(2 / np.pi)) < 1e-3 and (s >= 0).all()
    assert abs((bb + 8 * s).std() - 0.002) < 3e-4
    codes = (a[: off["gate_s"]].view(np.uint32)[:, None] >> (4 * np.arange(8, dtype=np.uint32))) & 15
    assert abs(codes.mean() - 7.5) < 0.01
    c2 = synth.expert_blob((1, 3), 4096, 1024, 2)
    off2, size2 = expert_offsets(4096, 1024, 64, 2)
    assert c2.size == size2 == 3932160
    s2 = synth.bf16_to_f32(c2[off2["gate_s"]: off2["gate_b"]].view(np.uint16))
    b2 = synth.bf16_to_f32(c2[off2["gate_b"]: off2["up_w"]].view(np.uint16))
    assert np.allclose(b2, -1.5 * s2, rtol=1e-2)
    x = synth.hidden_vec(synth.rng_for(0), 4096)
    assert np.array_equal(synth.bf16_round(x), x)


def test_zipf_routing_is_skewed(orc):
    rng = synth.rng_for(3)
    lg = synth.zipf_logits(rng, 512, 512)
    idx, _ = orc.route(lg, 10)
    counts = np.bincount(idx.reshape(-1), minlength=512)
    assert counts.max() > 300 and np.median(counts[counts > 0]) < 10


def test_workspace_status_rejects_null():
    L = fmoe_amd.lib()
    v = ctypes.c_uint32()
    assert L.fm_workspace_status(None, ctypes.byref(v), None) == -1
    assert b"NULL" in L.fm_last_error()


def test_prefill_workspace_covers_few_token_decode():
    """fm_prefill_moe runs 2-8 tokens (K <= 16) as one decode launch over all
    T x (K + shared) slots; its workspace query must leave room for that
    launch's hand-off buffers (status word + per-slot activations and outputs)."""
    L = fmoe_amd.lib()
    pool = fmoe_amd.ExpertPool(None, None, 512, 4096, 1024, 64)
    L.fm_prefill_moe_workspace_size.restype = ctypes.c_size_t
    L.fm_moe_decode_workspace_size.restype = ctypes.c_size_t
    for T in range(1, 10):
        for K in (1, 4, 10, 16):
            pf = L.fm_prefill_moe_workspace_size(T, K, ctypes.byref(pool), 0)
            need = L.fm_moe_decode_workspace_size(T * (K + 1), 4096, 1024)
            # hand-off buffers: 8-byte tagged words per activation and per output row
            assert need >= T * (K + 1) * (1024 + 4096) * 8
            if T <= 8:
                assert pf >= need, (T, K)


def test_c_consumer_compiles_and_links(tmp_path):
    """A C program that includes only include/*.h (and the HIP runtime API) and
    links -lfmoe with --no-undefined: every entry point it calls resolves in
    libfmoe.so.  Run without arguments it stops before any GPU call."""
    import subprocess
    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(here)
    exe = tmp_path / "fm_consumer"
    cmd = ["gcc", "-O2", "-std=c11", "-Wall", "-Werror", f"-I{root}/include", "-I/opt/rocm/include",
           "-D__HIP_PLATFORM_AMD__", os.path.join(here, "c_consumer", "fm_consumer.c"), "-o", str(exe),
           f"-L{root}/flash-moe_amd/lib", "-lfmoe", f"-Wl,-rpath,{root}/flash-moe_amd/lib", "-L/opt/rocm/lib",
           "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib", "-Wl,--no-undefined"]
    subprocess.run(cmd, check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 2 and "usage" in r.stderr


def test_moe_forward_checked_rejects_before_launch():
    """fm_moe_forward_checked validates its arguments on the host: a NULL
    status pointer or an incomplete layer is refused before any GPU call."""
    L = fmoe_amd.lib()
    layer = fmoe_amd.MoeLayer()
    st = ctypes.c_uint32(0)
    assert L.fm_moe_forward_checked(ctypes.byref(layer), 8, 1, 1, 1, None, 1, 1 << 20, None, None) == -1
    assert "NULL status" in L.fm_last_error().decode()
    assert L.fm_moe_forward_checked(ctypes.byref(layer), 8, 1, 1, 1, None, 1, 1 << 20, None, ctypes.byref(st)) == -1
    assert "incomplete layer" in L.fm_last_error().decode()
