"""CPU checks of the drop-in boundary: librnn.so loads (no GPU call is made),
exports every symbol include/rnn.h declares, and the product package never
touches the oracle; host-side validation raises like the reference panics."""
import os
import re
import subprocess

import pytest

import rustnn_amd

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_header_declares_the_abi():
    names = rustnn_amd.declared_symbols()
    for must in ("rnn_matmul", "rnn_gemm_small_batched", "rnn_matmul_dw", "rnn_conv2d_forward",
                 "rnn_conv2d_backward_w", "rnn_conv2d_backward_x", "rnn_attn_forward",
                 "rnn_attn_backward", "rnn_rel_index", "rnn_linear_forward",
                 "rnn_linear_backward", "rnn_dbg_im2col", "rnn_dbg_pack_a", "rnn_dbg_pack_b",
                 "rnn_dbg_rel_index", "rnn_ctx_create", "rnn_ctx_destroy"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = rustnn_amd.lib()  # loads librnn.so; nothing here initialises the GPU
    out = subprocess.run(["nm", "-D", "--defined-only", rustnn_amd.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\sT\s(rnn_\w+)", out))
    for name in rustnn_amd.declared_symbols():
        assert name in exported, name
        assert hasattr(lib, name)


def test_library_is_gfx950_only():
    """The offload bundle of our own build names gfx950 and no other target."""
    data = open(rustnn_amd.LIB_PATH, "rb").read()
    targets = set(re.findall(rb"amdgcn-amd-amdhsa--(gfx[0-9a-z]+)", data))
    assert targets == {b"gfx950"}, targets


def test_host_helpers_without_gpu():
    idx, nrel = rustnn_amd.rel_index(8, 8, 8, 8)
    assert nrel == 225 and idx.size == 4096 and int(idx.max()) < 225
    sp = rustnn_amd.ConvSpec.make(32, 64, 3, 2, 1, 32, 32)
    assert (sp.oh, sp.ow, sp.ckk, sp.hw) == (16, 16, 288, 256)
    with pytest.raises(ValueError):
        rustnn_amd.ConvSpec.make(3, 4, 9, 1, 0, 4, 4)  # k > h + 2*pad
    assert rustnn_amd.lib().rnn_status_string(-5).decode() == "unsupported shape"


def test_null_context_is_rejected():
    L = rustnn_amd.lib()
    assert L.rnn_matmul(None, 1, 1, 1, None, 0, None, 0, None, 0) == rustnn_amd.RNN_E_NULL
    assert L.rnn_conv2d_forward(None, None, 1, None, None, None) == rustnn_amd.RNN_E_NULL


def test_product_never_loads_the_oracle():
    pkg = os.path.join(ROOT, "rustnn_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                txt = open(os.path.join(dirpath, f)).read()
                assert "pyorc" not in txt and "liborc" not in txt and "import oracle" not in txt, f
