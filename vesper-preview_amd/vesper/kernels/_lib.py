"""ctypes binding of ``libvesper_kernels.so``: the one place Python meets the C ABI.

The library is the product path. It is loaded from this directory only; when it is missing or its
ABI version differs, every kernel call raises ``KernelLibraryError`` - there is no fallback. torch
is imported first so that its HIP runtime (``libamdhip64.so.7``) is the one the library binds to,
and the streams handed over are torch's.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
LIBRARY_PATH = HERE / "libvesper_kernels.so"
HEADER_PATH = HERE.parents[2] / "include" / "vesper_kernels.h"
ABI_VERSION = 20

P = ctypes.c_void_p
I = ctypes.c_int
Z = ctypes.c_size_t
F = ctypes.c_float
L = ctypes.c_int64

# every entry point of include/vesper_kernels.h: (return type, argument types)
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "vsp_last_error": (ctypes.c_char_p, []),
    "vsp_abi_version": (I, []),
    "vsp_init": (I, []),
    "vsp_fault_bits": (ctypes.c_uint, []),
    "vsp_clear_faults": (None, []),
    "vsp_set_wait_limit": (I, [I]),
    "vsp_set_scan_segments": (I, [I]),
    "vsp_delta_scan_workspace_bytes": (Z, [I, I, I, I, I]),
    "vsp_delta_scan_bf16": (I, [P, P, P, P, P, P, P, P, Z, P, I, I, I, I, P]),
    "vsp_delta_scan_f32": (I, [P, P, P, P, P, P, P, P, Z, P, I, I, I, I, P]),
    "vsp_delta_scan_records_bytes": (Z, [I, I, I, I]),
    "vsp_delta_scan_record_bf16": (I, [P, P, P, P, P, P, P, P, Z, P, P, Z, I, I, I, I, P]),
    "vsp_delta_scan_carried_bf16": (I, [P, P, P, P, P, P, P, P, P, P, P, Z, P, I, I, I, I, P]),
    "vsp_delta_scan_carried_f32": (I, [P, P, P, P, P, P, P, P, P, P, P, Z, P, I, I, I, I, P]),
    "vsp_delta_scan_logits_bf16": (I, [P, P, P, P, P, F, P, P, P, P, Z, P, I, I, I, I, P]),
    "vsp_delta_scan_logits_f32": (I, [P, P, P, P, P, F, P, P, P, P, Z, P, I, I, I, I, P]),
    "vsp_write_strength_bf16": (I, [P, P, F, P, I, I, P]),
    "vsp_write_strength_f32": (I, [P, P, F, P, I, I, P]),
    "vsp_delta_step_f32": (I, [P, P, P, P, P, P, P, P, I, I, I, P]),
    "vsp_delta_step_bf16": (I, [P, P, P, P, P, P, P, P, I, I, I, P]),
    "vsp_window_attn_bf16": (I, [P, P, P, P, P, I, I, I, I, I, I, I, F, P]),
    "vsp_window_attn_f16": (I, [P, P, P, P, P, I, I, I, I, I, I, I, F, P]),
    "vsp_delta_scan_backward_workspace_bytes": (Z, [I, I, I, I]),
    "vsp_delta_scan_backward_bf16": (I, [P, P, P, P, P, P, P, P, P, P, P, P, P, P, Z, I, I, I, I, P]),
    "vsp_delta_scan_backward_f32": (I, [P, P, P, P, P, P, P, P, P, P, P, P, P, P, Z, I, I, I, I, P]),
    "vsp_delta_scan_backward_recorded_bf16": (I, [P, P, P, P, P, P, P, P, P, Z, P, P, P, P, P, P, Z, I, I, I, I, P]),
    "vsp_window_attn_lse_bf16": (I, [P, P, P, P, P, P, I, I, I, I, I, I, I, F, P]),
    "vsp_window_attn_lse_f16": (I, [P, P, P, P, P, P, I, I, I, I, I, I, I, F, P]),
    "vsp_window_attn_carried_bf16": (I, [P, P, P, P, P, P, P, I, I, I, I, I, I, I, F, P]),
    "vsp_window_attn_carried_f16": (I, [P, P, P, P, P, P, P, I, I, I, I, I, I, I, F, P]),
    "vsp_window_attn_cached_bf16": (I, [P, P, P, P, P, P, P, I, I, I, I, I, I, I, F, P]),
    "vsp_window_attn_cached_f16": (I, [P, P, P, P, P, P, P, I, I, I, I, I, I, I, F, P]),
    "vsp_window_attn_backward_bf16": (I, [P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, I, I, F, P]),
    "vsp_window_attn_backward_f16": (I, [P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, I, I, F, P]),
    "vsp_ring_attn_workspace_bytes": (Z, [I]),
    "vsp_ring_attn_bf16": (I, [P, P, P, P, P, P, P, P, P, P, P, Z, I, I, I, I, I, F, I, P]),
    "vsp_ring_attn_f16": (I, [P, P, P, P, P, P, P, P, P, P, P, Z, I, I, I, I, I, F, I, P]),
    "vsp_ring_attn_bf16_ring_f32": (I, [P, P, P, P, P, P, P, P, P, P, P, Z, I, I, I, I, I, F, I, P]),
    "vsp_ring_attn_f16_ring_f32": (I, [P, P, P, P, P, P, P, P, P, P, P, Z, I, I, I, I, I, F, I, P]),
    "vsp_ring_attn_noalloc_bf16": (I, [P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, F, I, P]),
    "vsp_key_filter_bf16": (I, [P, P, P, P, I, I, I, I, I, P]),
    "vsp_key_filter_f16": (I, [P, P, P, P, I, I, I, I, I, P]),
    "vsp_key_filter_f32": (I, [P, P, P, P, I, I, I, I, I, P]),
    "vsp_key_step_bf16": (I, [P, P, P, P, P, P, P, I, I, I, I, I, P]),
    "vsp_key_step_f16": (I, [P, P, P, P, P, P, P, I, I, I, I, I, P]),
    "vsp_key_step_f32": (I, [P, P, P, P, P, P, P, I, I, I, I, I, P]),
    "vsp_copy_rows_where": (I, [I, P, P, P, P, I, P]),
    "vsp_kv_cache_push": (I, [P, P, P, P, P, P, P, P, P, I, I, I, I, I, I, I, P]),
    "vsp_rotary_qk_bf16": (I, [P, P, P, P, P, P, I, I, I, I, I, P]),
    "vsp_rotary_qk_f16": (I, [P, P, P, P, P, P, I, I, I, I, I, P]),
    "vsp_rotary_qk_f32": (I, [P, P, P, P, P, P, I, I, I, I, I, P]),
    "vsp_rms_norm_bf16": (I, [P, P, P, I, I, P]),
    "vsp_add_rms_norm_bf16": (I, [P, P, P, P, P, I, I, P]),
    "vsp_halt_step": (I, [P, P, P, P, P, I, P]),
    "vsp_residual_rows_where": (I, [P, P, P, P, I, I, P]),
    "vsp_delta_step_keys_bf16": (I, [P, P, P, P, P, P, I, P, P, P, P, I, I, I, P]),
    "vsp_decode_proj_bf16": (I, [P, P, P, P, P, I, I, I, I, I, I, I, I, P, P, P, P, I, P, P, I, I, P]),
    "vsp_project_bf16": (I, [P, P, I, I, I, I, I, I, I, I, P, P, P, P, I, P]),
    "vsp_key_filter_backward_workspace_bytes": (Z, [I, I, I, I]),
    "vsp_key_filter_backward_bf16": (I, [P, P, P, P, P, P, P, P, Z, I, I, I, I, I, P]),
    "vsp_key_filter_backward_f16": (I, [P, P, P, P, P, P, P, P, Z, I, I, I, I, I, P]),
    "vsp_key_filter_backward_f32": (I, [P, P, P, P, P, P, P, P, Z, I, I, I, I, I, P]),
    "vsp_normalize_keys_bf16": (I, [P, P, L, I, P]),
    "vsp_normalize_keys_f16": (I, [P, P, L, I, P]),
    "vsp_normalize_keys_f32": (I, [P, P, L, I, P]),
    "vsp_normalize_keys_backward_bf16": (I, [P, P, P, L, I, P]),
    "vsp_normalize_keys_backward_f16": (I, [P, P, P, L, I, P]),
    "vsp_normalize_keys_backward_f32": (I, [P, P, P, L, I, P]),
}


class KernelLibraryError(RuntimeError):
    """The HIP kernel library is missing, stale, or a kernel call failed."""


_LIB: ctypes.CDLL | None = None


def library() -> ctypes.CDLL:
    """The loaded library with every signature declared; raises if it is not built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIBRARY_PATH.exists():
        raise KernelLibraryError(
            f"{LIBRARY_PATH} is not built: run `python -m vesper.kernels.build` (or __graft_entry__.build())"
        )
    lib = ctypes.CDLL(str(LIBRARY_PATH))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = lib.vsp_abi_version()
    if version != ABI_VERSION:
        raise KernelLibraryError(f"{LIBRARY_PATH} has ABI {version}, this package needs {ABI_VERSION}")
    if torch.cuda.is_available() and lib.vsp_init() != 0:
        raise KernelLibraryError(f"vsp_init failed: {lib.vsp_last_error().decode('utf-8', 'replace')}")
    _LIB = lib
    return lib


FAULT_NAMES = {0: "the bf16 scan's chunk hand-over"}


def check_faults(synchronize: bool = False) -> None:
    """Raise ``KernelLibraryError`` if a kernel's bounded wait has given up since the last
    ``clear_faults`` (its outputs from then on are NaN). Without ``synchronize`` it sees kernels
    that have completed; with it, every kernel queued on the current device so far."""
    lib = library()
    if synchronize and torch.cuda.is_available():
        torch.cuda.synchronize()
    bits = lib.vsp_fault_bits()
    if bits:
        names = ", ".join(FAULT_NAMES.get(i, f"kernel family {i}") for i in range(32) if bits >> i & 1)
        raise KernelLibraryError(f"a bounded wait gave up in {names}: its results are invalid (NaN); "
                                 "clear_faults() resets the record")


def clear_faults() -> None:
    library().vsp_clear_faults()


def set_wait_limit(polls: int) -> int:
    """Polls a bounded wait makes before giving up (negative: the default); returns the previous."""
    return int(library().vsp_set_wait_limit(polls))


def set_scan_segments(form: int) -> int:
    """The form of the bf16 scan at head width 64: 0 (or False) value-slice chains over the whole
    sequence, 1 (or True) segments joined by their affine maps, 2 by shape (the default); returns
    the previous setting."""
    return int(library().vsp_set_scan_segments(int(form)))


def available() -> bool:
    """Whether the library loads (it does on a machine without a GPU too)."""
    try:
        library()
    except (KernelLibraryError, OSError):
        return False
    return True


def header_symbols() -> list[str]:
    """The function names declared in ``include/vesper_kernels.h``."""
    text = HEADER_PATH.read_text(encoding="utf-8")
    return sorted(set(re.findall(r"\b(vsp_[a-z0-9_]+)\s*\(", text)))


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(device: torch.device) -> int:
    """torch's current stream on ``device`` as a hipStream_t handle."""
    return torch.cuda.current_stream(device).cuda_stream


def call(name: str, *args: object) -> None:
    """Call an entry point and turn a nonzero status into ``KernelLibraryError``."""
    lib = library()
    if lib.vsp_fault_bits():  # a fault of an earlier call: its results, and what used them, are invalid
        check_faults()
    status = getattr(lib, name)(*args)
    if status != 0:
        message = lib.vsp_last_error().decode("utf-8", "replace")
        raise KernelLibraryError(f"{name} returned {status}: {message}")
