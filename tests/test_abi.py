"""C-ABI checks that need no GPU: exports, struct layout, argument validation.

No kernel is launched here; every call below returns from the host-side
validation in libaffmae.so before any HIP API is used.
"""
import ctypes
import re
import subprocess
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "affmae.h"

from affmae_amd import _lib  # noqa: E402


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(aff_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_library_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert "aff_knn" in names and "aff_nbhd_attn_fwd" in names
    for n in names:
        assert hasattr(lib, n), f"{n} declared in affmae.h but not exported"
    # and the ctypes table covers exactly the header
    assert sorted(_lib.SIGNATURES) == names


def test_abi_version(lib):
    assert lib.aff_abi_version() == _lib.ABI_VERSION


@pytest.mark.parametrize("cname,cls", [("aff_nbhd_attn_args", "NbhdAttnArgs"), ("aff_nbhd_attn_bwd_args", "NbhdAttnBwdArgs"),
                                       ("aff_deform_args", "DeformArgs"), ("aff_deform_bwd_args", "DeformBwdArgs"),
                                       ("aff_sfc_curve_args", "SfcCurveArgs"), ("aff_sfc_anchor_args", "SfcAnchorArgs")])
def test_struct_layout_matches_header(tmp_path, cname, cls):
    """Size and every field offset of the ctypes mirror equal the C struct's (gcc on the header)."""
    struct = getattr(_lib, cls)
    fields = [f for f, _ in struct._fields_]
    src = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"', "int main(void){",
           f'printf("%zu\\n", sizeof({cname}));']
    src += [f'printf("%zu\\n", offsetof({cname}, {f}));' for f in fields]
    src += ["return 0;}"]
    c = tmp_path / "probe.c"
    c.write_text("\n".join(src))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", str(c), "-o", str(exe)], check=True)
    vals = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert vals[0] == ctypes.sizeof(struct)
    assert len(vals) == len(fields) + 1
    for f, off in zip(fields, vals[1:]):
        assert getattr(struct, f).offset == off, f


DUMMY = 0x10000  # never dereferenced: validation fails first


def test_knn_validation(lib):
    ws = lib.aff_knn_workspace_bytes(2, 10, 20, 2, 4)
    assert ws > 0
    # k > N
    st = lib.aff_knn(DUMMY, 20, 2, DUMMY, 40, 2, 2, 10, 20, 2, 21, DUMMY, 0, None, DUMMY, ws, None)
    assert st == _lib.AFF_ERR_INVALID_ARG
    assert b"exceeds number of reference points" in lib.aff_last_error()
    # unsupported D, and k > 64 outside 2-D
    st = lib.aff_knn(DUMMY, 50, 5, DUMMY, 100, 5, 2, 10, 20, 5, 4, DUMMY, 0, None, DUMMY, ws, None)
    assert st == _lib.AFF_ERR_UNSUPPORTED
    assert lib.aff_knn_workspace_bytes(2, 10, 100, 3, 65) == 0
    st = lib.aff_knn(DUMMY, 300, 3, DUMMY, 300, 3, 2, 10, 100, 3, 65, DUMMY, 0, None, None, 0, None)
    assert st == _lib.AFF_ERR_UNSUPPORTED
    # missing / short workspace
    st = lib.aff_knn(DUMMY, 20, 2, DUMMY, 40, 2, 2, 10, 20, 2, 4, DUMMY, 0, None, None, 0, None)
    assert st == _lib.AFF_ERR_WORKSPACE
    st = lib.aff_knn(DUMMY, 20, 2, DUMMY, 40, 2, 2, 10, 20, 2, 4, DUMMY, 0, None, DUMMY, ws - 1, None)
    assert st == _lib.AFF_ERR_WORKSPACE
    # empty problems are a no-op
    assert lib.aff_knn(None, 0, 0, None, 0, 0, 0, 10, 20, 2, 4, None, 0, None, None, 0, None) == _lib.AFF_OK
    assert lib.aff_knn(None, 0, 0, None, 0, 0, 2, 0, 20, 2, 4, None, 0, None, None, 0, None) == _lib.AFF_OK


def _args(**kw):
    a = _lib.NbhdAttnArgs()
    a.dtype, a.B, a.H, a.N, a.M, a.D, a.scale = _lib.AFF_BF16, 1, 2, 16, 8, 32, 0.17
    for n in ("q", "k", "v", "out", "member_idx"):
        setattr(a, n, DUMMY)
    a.q_sb = a.k_sb = a.v_sb = a.o_sb = 2 * 16 * 32
    a.q_sh = a.k_sh = a.v_sh = a.o_sh = 16 * 32
    a.q_sn = a.k_sn = a.v_sn = a.o_sn = 32
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,code", [
    (dict(D=12), _lib.AFF_ERR_INVALID_ARG),
    (dict(D=24), _lib.AFF_ERR_UNSUPPORTED),
    (dict(dtype=7), _lib.AFF_ERR_UNSUPPORTED),
    (dict(bias_mode=5), _lib.AFF_ERR_INVALID_ARG),
    (dict(bias_mode=1), _lib.AFF_ERR_INVALID_ARG),        # no bias pointer
    (dict(bias_mode=2, pe_idx=DUMMY), _lib.AFF_ERR_INVALID_ARG),   # no table
    (dict(bias_mode=3, pos=DUMMY), _lib.AFF_ERR_INVALID_ARG),      # no weights
    (dict(blank_k=DUMMY), _lib.AFF_ERR_INVALID_ARG),      # blank_v missing
    (dict(q_sn=33), _lib.AFF_ERR_INVALID_ARG),            # row not 16-byte aligned
    (dict(q=DUMMY + 2), _lib.AFF_ERR_INVALID_ARG),        # pointer not 16-byte aligned
    (dict(member_idx=None), _lib.AFF_ERR_INVALID_ARG),
])
def test_attention_validation(lib, kw, code):
    a = _args(**kw)
    assert lib.aff_nbhd_attn_fwd(ctypes.byref(a), None) == code
    assert lib.aff_last_error()


def test_attention_null_and_empty(lib):
    assert lib.aff_nbhd_attn_fwd(None, None) == _lib.AFF_ERR_INVALID_ARG
    a = _args(N=0)
    assert lib.aff_nbhd_attn_fwd(ctypes.byref(a), None) == _lib.AFF_OK


def test_status_mapping(lib):
    with pytest.raises(ValueError):
        _lib.check(_lib.AFF_ERR_INVALID_ARG, "x")
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.AFF_ERR_UNSUPPORTED, "x")
    with pytest.raises(_lib.AffLaunchError):
        _lib.check(_lib.AFF_ERR_LAUNCH, "x")


# ----------------------------------------- Python wrappers (reference asserts) --
def test_wrappers_reject_cpu_tensors():
    from affmae_amd.kernels import knn, knn_forward, launch_flash_nbhood_attn_fwd
    p = torch.rand(1, 10, 2)
    with pytest.raises(AssertionError, match="Inputs must be on CUDA"):
        knn_forward(p, p, 4)
    with pytest.raises(AssertionError, match="Inputs must be on CUDA"):
        knn(p, p, 4)
    q = torch.rand(1, 2, 16, 32)
    idx = torch.zeros(1, 16, 8, dtype=torch.int64)
    with pytest.raises(AssertionError, match="Inputs must be on CUDA"):
        launch_flash_nbhood_attn_fwd(q, q, q, idx, 0.2)


def test_wrapper_shape_asserts():
    from affmae_amd.kernels import launch_flash_nbhood_attn_fwd
    q = torch.rand(1, 2, 16, 12)
    idx = torch.zeros(1, 16, 8, dtype=torch.int64)
    with pytest.raises(AssertionError, match="head_dim must be a multiple of 8"):
        launch_flash_nbhood_attn_fwd(q, q, q, idx, 0.2)
    q = torch.rand(1, 2, 16, 32)
    with pytest.raises(AssertionError, match="neighbor_size must be a multiple of 8"):
        launch_flash_nbhood_attn_fwd(q, q, q, torch.zeros(1, 16, 6, dtype=torch.int64), 0.2)
    with pytest.raises(AssertionError, match="same shape"):
        launch_flash_nbhood_attn_fwd(q, q[..., :16], q, idx, 0.2)


def test_pre_table_matches_oracle(oracle_mod):
    from affmae_amd.utils.pos_embed import pre_table_fp32
    import numpy as np
    np.testing.assert_allclose(pre_table_fp32.numpy(), oracle_mod.pre_table(), rtol=1e-6, atol=1e-6)


def test_fused_knn_config_matches_launch():
    """The reported launch shape follows aff_deform_fwd: cfg4 (4 levels x 4 points,
    3 neighbours, C=32) takes 16 rows per wave and 24 576 bytes of LDS per 4-wave
    workgroup, the figure the kernel trace records for deform_cand_kernel."""
    from affmae_amd.kernels.fused_deform_attn import get_fused_knn_config
    c = get_fused_knn_config(32, 12544, 8, 4, 32, L=4, knn_k=3)
    assert c["rows_per_wave"] == 16 and c["lanes_per_row_search"] == 4
    assert c["waves_per_workgroup"] == 4 and c["lds_bytes_per_workgroup"] == 24576
    assert c["workgroups"] == 32 * 12544 * 8 // 64
    assert c["lanes_per_row_gather"] == 4 and c["gather_rows_in_flight"] == 8
    one = get_fused_knn_config(2, 1000, 6, 1, 64)
    assert one["rows_per_wave"] == 64 and one["lanes_per_row_search"] == 1
    with pytest.raises(ValueError):
        get_fused_knn_config(0, 1, 1, 1, 1)
