"""CPU checks of the boundary: the C-ABI library loads and exports what its header declares, and
the Python entry points refuse what the contract excludes before any kernel runs."""

from __future__ import annotations

import pytest
import torch

BF16 = torch.bfloat16


def test_the_library_exports_every_declared_symbol():
    from vesper.kernels import _lib

    lib = _lib.library()
    declared = _lib.header_symbols()
    assert "vsp_delta_scan_bf16" in declared and "vsp_last_error" in declared
    for name in declared:
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert lib.vsp_abi_version() == _lib.ABI_VERSION


def test_the_library_never_switches_devices():
    """The library works on the caller's current device only: it imports no HIP call that changes
    or enumerates devices, so loading it (vsp_init) and calling any entry point cannot create a
    context on another GPU."""
    import shutil
    import subprocess

    from vesper.kernels import _lib

    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("binutils' nm is not installed")
    out = subprocess.run([nm, "-D", "--undefined-only", str(_lib.LIBRARY_PATH)], capture_output=True, text=True,
                         check=True).stdout
    imported = {line.split()[-1].split("@")[0] for line in out.splitlines() if line.strip()}
    assert "hipGetDevice" in imported  # the check sees the HIP imports at all
    for call in ("hipSetDevice", "hipGetDeviceCount", "hipDeviceReset", "hipDevicePrimaryCtxRetain"):
        assert call not in imported, call


def test_the_workspace_size_covers_every_chunk():
    from vesper.kernels import _lib

    lib = _lib.library()
    # ten 16x16 lower tiles of the UT factor per 64-token chunk; the bf16 scan at width 64 adds, per
    # head, the affine maps (X and M, fp32 [64, 64] each) of every segment but the last and a copy of
    # S0: at B8 H8 four segments of sixteen chunks, at B1 H2 T4096 sixteen of four, at B2 H1 T520 two
    # of five, and none where a head has fewer than eight chunks or B H reaches 256
    seg = lambda heads, maps: heads * (maps * 2 + 1) * 64 * 64 * 4  # noqa: E731
    assert lib.vsp_delta_scan_workspace_bytes(8, 4096, 8, 64, 0) == 8 * 8 * 64 * 2560 * 2 + seg(64, 3)
    assert lib.vsp_delta_scan_workspace_bytes(1, 4096, 2, 64, 0) == 2 * 64 * 2560 * 2 + seg(2, 15)
    assert lib.vsp_delta_scan_workspace_bytes(2, 520, 1, 64, 0) == 2 * 9 * 2560 * 2 + seg(2, 1)
    assert lib.vsp_delta_scan_workspace_bytes(1, 300, 1, 64, 0) == 5 * 2560 * 2
    assert lib.vsp_delta_scan_workspace_bytes(32, 4096, 8, 64, 0) == 32 * 8 * 64 * 2560 * 2
    assert lib.vsp_delta_scan_workspace_bytes(8, 4096, 8, 32, 0) == 8 * 8 * 64 * 2560 * 2
    assert lib.vsp_delta_scan_workspace_bytes(2, 130, 3, 16, 1) == 2 * 3 * 3 * 2560 * 4
    assert lib.vsp_delta_scan_workspace_bytes(2, 130, 3, 128, 1) == 0  # fp32 at 128 runs token by token
    assert lib.vsp_delta_scan_workspace_bytes(2, 130, 3, 48, 1) == 0  # token-serial width
    assert lib.vsp_delta_scan_workspace_bytes(2, 10, 3, 64, 0) == 0  # short sequences are serial
    # the backward: six [D, D] blocks and one [64, 64] block a chunk on the tiled widths; the wide
    # backward keeps per head a [D, D] state a chunk, the state's gradient and the final state, and
    # per chunk three [64, 64] blocks (L, P, the Gram matrix) and per value group of 64 columns two
    # [64, 64] and two [64, D] partial sums
    tiled = 2 * 3 * 3 * (64 * 64 + 6 * 64 * 64) * 4
    assert lib.vsp_delta_scan_backward_workspace_bytes(2, 130, 3, 64) == tiled
    wide = 2 * ((3 + 2) * 192 * 192 + 3 * (3 * 64 * 64 + 3 * (2 * 64 * 64 + 2 * 64 * 192))) * 4
    assert lib.vsp_delta_scan_backward_workspace_bytes(1, 130, 2, 192) == wide
    assert lib.vsp_delta_scan_backward_workspace_bytes(1, 130, 2, 128) == 2 * 3 * (64 * 64 + 6 * 128 * 128) * 4
    assert lib.vsp_delta_scan_backward_workspace_bytes(1, 130, 2, 200) == 0  # not a multiple of 16
    assert lib.vsp_delta_scan_backward_workspace_bytes(1, 130, 2, 272) == 0  # above 256
    assert lib.vsp_ring_attn_workspace_bytes(64) == 64 * 4  # one arrival counter per row
    assert lib.vsp_ring_attn_workspace_bytes(0) == 0


def test_a_bad_size_is_an_error_status_not_a_crash():
    from vesper.kernels import _lib

    lib = _lib.library()
    status = lib.vsp_delta_scan_f32(None, None, None, None, None, None, None, None, 0, None, 1, 8, 1, 300, None)
    assert status == 1
    assert "head dimension 300" in lib.vsp_last_error().decode()


def test_refuses_a_cpu_tensor_before_touching_the_kernel():
    from vesper.contracts import ContractError
    from vesper.kernels.delta_scan import delta_scan_fused, delta_scan_fused_fp32, delta_scan_step_fused

    z = torch.zeros(1, 4, 1, 8, dtype=BF16)
    with pytest.raises(ContractError, match="CUDA only"):
        delta_scan_fused(z, z, z, torch.zeros(1, 4, 1, dtype=BF16), torch.zeros(1, 1, 8, 8))
    z = torch.zeros(1, 4, 1, 8)
    with pytest.raises(ContractError, match="CUDA only"):
        delta_scan_fused_fp32(z, z, z, torch.zeros(1, 4, 1), torch.zeros(1, 1, 8, 8))
    z = torch.zeros(1, 1, 8)
    with pytest.raises(ContractError, match="CUDA only"):
        delta_scan_step_fused(z, z, z, torch.zeros(1, 1), torch.zeros(1, 1, 8, 8))


def test_shape_and_dtype_refusals_come_first():
    from vesper.contracts import ContractError
    from vesper.kernels.delta_scan import MAX_HEAD_DIM, delta_scan_fused

    assert MAX_HEAD_DIM == 256
    z = torch.zeros(1, 4, 1, 8, dtype=BF16)
    with pytest.raises(ContractError, match="dtype"):
        delta_scan_fused(z.float(), z, z, torch.zeros(1, 4, 1, dtype=BF16), torch.zeros(1, 1, 8, 8))
    with pytest.raises(ContractError, match="axis"):
        delta_scan_fused(z, z[:, :2], z, torch.zeros(1, 4, 1, dtype=BF16), torch.zeros(1, 1, 8, 8))


def test_the_product_path_does_not_import_the_oracle():
    import subprocess
    import sys

    from conftest import PACKAGE_ROOT

    code = (
        "import sys; sys.path.insert(0, %r); import vesper.kernels.delta_scan, vesper.kernels._lib; "
        "print(any(m == 'oracle' or m.startswith('oracle.') for m in sys.modules))" % str(PACKAGE_ROOT)
    )
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, check=True)
    assert out.stdout.strip() == "False"


def test_the_scan_switch_refuses_what_it_cannot_run():
    # the reference's names and refusals (vesper/column.py:382-426): "reference" runs anywhere but
    # not captured on the GPU; the fused scans need the GPU
    from vesper.column import SCAN_IMPLS, check_capturable_scan, check_scan

    assert SCAN_IMPLS == ("reference", "fused", "fused-fp32")
    assert check_scan("reference", torch.device("cpu")) == "reference"
    assert check_scan("reference", torch.device("cuda")) == "reference"
    assert check_capturable_scan("reference", torch.device("cpu")) == "reference"
    with pytest.raises(ValueError, match="cannot run as a captured graph"):
        check_capturable_scan("reference", torch.device("cuda"))
    with pytest.raises(ValueError, match="must be one of"):
        check_scan("triton", torch.device("cpu"))
    with pytest.raises(ValueError, match="needs the model on CUDA"):
        check_scan("fused", torch.device("cpu"))
    with pytest.raises(ValueError, match="needs the model on CUDA"):
        check_capturable_scan("fused-fp32", torch.device("cpu"))


def test_the_key_filter_refuses_before_launching():
    from vesper.contracts import ContractError
    from vesper.kernels import _lib
    from vesper.kernels.keys import fused_keys

    z = torch.zeros(1, 4, 128)
    taps = torch.ones(4, 128)
    with pytest.raises(ContractError, match="CUDA only"):
        fused_keys(z, torch.zeros(1, 3, 128), taps, 2)
    with pytest.raises(ContractError, match="dtype"):
        fused_keys(z.double(), torch.zeros(1, 3, 128), taps, 2)
    with pytest.raises(ContractError, match="axis"):
        fused_keys(z, torch.zeros(1, 4, 128), taps, 2)
    lib = _lib.library()
    assert lib.vsp_key_filter_bf16(None, None, None, None, 1, 4, 128, 2, 9, None) == 2  # unsupported
    assert "filter width 9" in lib.vsp_last_error().decode()
    assert lib.vsp_key_filter_f32(None, None, None, None, 1, 4, 128, 32, 4, None) == 2
    assert "head width 4" in lib.vsp_last_error().decode()
    assert lib.vsp_key_filter_f16(None, None, None, None, 1, 4, 128, 2, 4, None) == 1  # bad argument
    assert "null pointer" in lib.vsp_last_error().decode()
    assert lib.vsp_key_filter_bf16(None, None, None, None, 0, 4, 128, 2, 4, None) == 0  # nothing to do
    # the key step's next history may not overlap the history it is computed from (refused before
    # any launch: the addresses are only compared)
    base = 1 << 20
    assert lib.vsp_key_step_bf16(base, None, None, base + 4096, base + 8192, base + 12288, base + 4096 + 16,
                                 1, 4, 128, 2, 4, None) == 1
    assert "overlaps the history" in lib.vsp_last_error().decode()
    assert lib.vsp_key_step_bf16(base, base + 64, None, base + 4096, base + 8192, base + 12288, None,
                                 1, 4, 128, 2, 4, None) == 1
    assert "active flags" in lib.vsp_last_error().decode()


def test_set_scan_and_scan_of_over_a_model():
    # column.py:353-380, :428-441: one choice for every recurrent sublayer; refused before any change
    from torch import nn

    from vesper.column import RecurrentSublayer, scan_of, set_scan

    g = torch.Generator().manual_seed(0)
    model = nn.Sequential(RecurrentSublayer(32, 2, generator=g), nn.Linear(4, 4), RecurrentSublayer(32, 2, generator=g))
    assert scan_of(model) == "reference"
    assert set_scan(model, "reference") == 2
    with pytest.raises(ValueError, match="needs the model on CUDA"):
        set_scan(model, "fused")
    assert scan_of(model) == "reference"  # unchanged by the refused call
    with pytest.raises(ValueError, match="must be one of"):
        set_scan(model, "triton")
    with pytest.raises(ValueError, match="no recurrent sublayer"):
        set_scan(nn.Linear(4, 4), "reference")
    model[2].scan_impl = "fused"
    with pytest.raises(ValueError, match="expected exactly one"):
        scan_of(model)
    with pytest.raises(ValueError, match="expected exactly one"):
        scan_of(nn.Linear(4, 4))


def test_the_reference_scan_backend_equals_the_oracle_scan():
    # the "reference" choice of RecurrentSublayer.scan (column.py:316-326): the chunked scan in the
    # promoted dtype, then W_o; checked against the oracle's chunked scan (itself pinned by the
    # reference's rational known answers) and against the token-serial recurrence
    from oracle.delta import delta_scan_chunked, delta_scan_serial, normalize_keys
    from vesper.column import RecurrentSublayer

    g = torch.Generator().manual_seed(1)
    layer = RecurrentSublayer(32, 2, block=8, generator=g).double()
    x = torch.randn(2, 21, 32, generator=g, dtype=torch.float64)
    q, z, v, beta = layer.project(x)
    k = normalize_keys(z.view(2, 21, 2, 16))
    s0 = 0.1 * torch.randn(2, 2, 16, 16, generator=g, dtype=torch.float64)
    y, s1 = layer.scan(q, k, v, beta, s0)
    o_ref, s_ref = delta_scan_chunked(q, k, v, beta, s0, 64)
    o_ser, s_ser = delta_scan_serial(q, k, v, beta, s0)
    torch.testing.assert_close(y, o_ref.flatten(2) @ layer.w_o.T, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(s1, s_ref, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(s1, s_ser, rtol=1e-10, atol=1e-10)
    # bf16 projections run the scan in float32, as the reference promotes them; the reads return
    # in the projections' dtype
    from vesper.column import recurrent_scan

    o16, s32 = recurrent_scan("reference", *(t.to(torch.bfloat16) for t in (q, k, v, beta)), s0.float())
    assert o16.dtype == torch.bfloat16 and s32.dtype == torch.float32
