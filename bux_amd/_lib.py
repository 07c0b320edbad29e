"""The HIP library, ``libbux_amd.so``, through ctypes: every entry point that
``include/bux_amd.h`` declares, with its argument types.

`load()` returns the library, building nothing: ``python -m bux_amd.build`` (or
``__graft_entry__.build()``) makes it. A missing library raises at once; there is no
fallback to another implementation. `check(rc)` turns a nonzero return code into a
`BuxError` carrying the library's message.
"""

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
PATH = os.path.join(HERE, "libbux_amd.so")

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_int = ctypes.c_int
_f32 = ctypes.c_float
_size = ctypes.c_size_t


class FfnStruct(ctypes.Structure):
    """``bux_ffn``: an expert FFN's activation settings."""

    _fields_ = [
        ("activation", ctypes.c_int32),
        ("gated", ctypes.c_int32),
        ("clamped", ctypes.c_int32),
        ("limit", ctypes.c_float),
        ("capped", ctypes.c_int32),
        ("up_softcap", ctypes.c_float),
        ("up_offset", ctypes.c_float),
    ]


_ffn = ctypes.POINTER(FfnStruct)


class NormStruct(ctypes.Structure):
    """``bux_norm``: the experts' output norm's settings."""

    _fields_ = [
        ("kind", ctypes.c_int32),
        ("affine", ctypes.c_int32),
        ("zero_centered", ctypes.c_int32),
        ("scale_input", ctypes.c_int32),
        ("bias", ctypes.c_int32),
        ("eps", ctypes.c_float),
    ]


_norm = ctypes.POINTER(NormStruct)

# name -> (restype, argtypes), as include/bux_amd.h declares them.
SIGNATURES = {
    "bux_last_error": (ctypes.c_char_p, []),
    "bux_version": (_int, []),
    "bux_moe_permute_workspace_size": (_size, [_i64, _i32]),
    "bux_moe_permute": (_int, [_p, _i64, _i32, _p, _p, _p, _p, _p, _size, _p]),
    "bux_mx_quantize": (
        _int, [_p, _p, _i32, _i64, _i64, _i64, _i64, _i64, _p, _int, _p, _p, _p, _p, _p]),
    "bux_mx_quantize_f32": (
        _int, [_p, _p, _i32, _i64, _i64, _i64, _i64, _i64, _p, _int, _p, _p, _p, _p, _p]),
    "bux_mx_grouped_rows_workspace_size": (_size, [_i32, _i64, _i64]),
    "bux_mx_grouped_rows": (
        _int, [_p, _p, _p, _p, _p, _i32, _i64, _i64, _i64, _i64, _int, _p, _p, _size, _p]),
    "bux_mx_grouped_rows_started": (
        _int, [_p, _p, _p, _p, _p, _p, _i32, _i64, _i64, _i64, _i64, _int, _p, _p, _size, _p]),
    "bux_mx_grouped_tiles": (_int, [_p, _i32, _i64, _i64, _p, _size, _p]),
    "bux_mx_grouped_rows_listed": (
        _int, [_p, _p, _p, _p, _p, _size, _i32, _i64, _i64, _i64, _i64, _int, _p, _p]),
    "bux_mx_grouped_contract_listed": (
        _int, [_p, _p, _p, _p, _p, _size, _i32, _i64, _i64, _i64, _int, _p, _p]),
    "bux_mx_grouped_rows_noalloc": (
        _int, [_p, _p, _p, _p, _p, _i32, _i64, _i64, _i64, _i64, _int, _p, _p]),
    "bux_mx_grouped_contract_workspace_size": (_size, [_i32]),
    "bux_mx_grouped_contract": (
        _int, [_p, _p, _p, _p, _p, _i32, _i64, _i64, _i64, _int, _p, _p, _size, _p]),
    "bux_bf16_grouped_rows_workspace_size": (_size, [_i32, _i64]),
    "bux_bf16_grouped_rows": (
        _int, [_p, _p, _int, _p, _i32, _i64, _i64, _i64, _p, _p, _size, _p]),
    "bux_bf16_grouped_contract_workspace_size": (_size, [_i32]),
    "bux_bf16_grouped_contract": (_int, [_p, _p, _p, _i32, _i64, _i64, _i64, _p, _p, _size, _p]),
    "bux_bf16_grouped_rows_f32": (
        _int, [_p, _p, _int, _p, _i32, _i64, _i64, _i64, _p, _p, _size, _p]),
    "bux_bf16_grouped_contract_f32": (_int, [_p, _p, _p, _i32, _i64, _i64, _i64, _p, _p, _size, _p]),
    "bux_token_rows": (_int, [_p, _i64, _p, _i64, _i32, _i64, _p, _p]),
    "bux_token_sums": (_int, [_p, _i64, _p, _i64, _i32, _i64, _p, _p]),
    "bux_token_sums_f32": (_int, [_p, _i64, _p, _i64, _i32, _i64, _p, _p]),
    "bux_token_sums_biased": (_int, [_p, _i64, _p, _i64, _i32, _i64, _p, _p, _i32, _p, _p, _p]),
    "bux_expert_bias_add": (_int, [_p, _i64, _i64, _p, _p, _i32, _p]),
    "bux_expert_sums": (_int, [_p, _p, _i32, _i64, _p, _i64, _i64, _p, _i32, _p, _p]),
    "bux_expert_bias_weight_grad": (_int, [_p, _p, _i32, _i64, _i64, _i64, _p, _p, _i32, _p, _p]),
    "bux_expert_norm_forward": (_int, [_p, _i64, _i64, _p, _p, _i32, _norm, _p, _p, _p, _p, _p]),
    "bux_expert_norm_backward_workspace_size": (_size, [_i64, _i64]),
    "bux_expert_norm_backward": (
        _int, [_p, _p, _i32, _i64, _p, _i64, _i64, _p, _p, _i32, _norm, _p, _p, _p, _p, _p, _p, _p,
               _p, _size, _p]),
    "bux_token_sums_biased_f32": (_int, [_p, _i64, _p, _i64, _i32, _i64, _p, _p, _i32, _p, _p, _p]),
    "bux_expert_bias_add_f32": (_int, [_p, _i64, _i64, _p, _p, _i32, _p]),
    "bux_expert_sums_f32": (_int, [_p, _p, _i32, _i64, _p, _i64, _i64, _p, _i32, _p, _p]),
    "bux_expert_bias_weight_grad_f32": (_int, [_p, _p, _i32, _i64, _i64, _i64, _p, _p, _i32, _p, _p]),
    "bux_expert_norm_forward_f32": (_int, [_p, _i64, _i64, _p, _p, _i32, _norm, _p, _p, _p, _p, _p]),
    "bux_expert_norm_backward_f32": (
        _int, [_p, _p, _i32, _i64, _p, _i64, _i64, _p, _p, _i32, _norm, _p, _p, _p, _p, _p, _p, _p,
               _p, _size, _p]),
    "bux_glu_forward": (_int, [_p, _p, _p, _i64, _i64, _ffn, _p, _p]),
    "bux_glu_backward": (_int, [_p, _p, _p, _p, _i64, _i64, _ffn, _p, _p, _p]),
    "bux_glu_forward_f32": (_int, [_p, _p, _p, _i64, _i64, _ffn, _p, _p]),
    "bux_glu_backward_f32": (_int, [_p, _p, _p, _p, _i64, _i64, _ffn, _p, _p, _p]),
    "bux_glu_quantize": (
        _int, [_p, _p, _p, _i64, _i64, _ffn, _i64, _p, _p, _p, _p, _p, _p]),
    "bux_glu_quantize_f32": (
        _int, [_p, _p, _p, _i64, _i64, _ffn, _i64, _p, _p, _p, _p, _p, _p]),
    "bux_mx_grouped_glu_workspace_size": (_size, [_i32, _i64]),
    "bux_mx_grouped_glu": (
        _int, [_p, _p, _p, _p, _p, _i32, _i64, _i64, _i64, _i64, _p, _ffn, _p, _p,
               _p, _p, _p, _p, _size, _p]),
    "bux_mx_grouped_dglu_workspace_size": (_size, [_i32, _i64, _i64, _i64]),
    "bux_mx_grouped_dglu": (
        _int, [_p, _p, _p, _p, _p, _i32, _i64, _i64, _i64, _i64, _p, _p, _ffn, _p, _p, _p, _p,
               _p, _p, _p, _size, _p]),
    "bux_glu_backward_quantize_workspace_size": (_size, [_i64, _i64]),
    "bux_glu_backward_quantize": (
        _int, [_p, _p, _p, _p, _i64, _i64, _ffn, _i64, _p, _p, _p, _p, _p, _p, _p,
               _size, _p]),
    "bux_glu_backward_quantize_f32": (
        _int, [_p, _p, _p, _p, _i64, _i64, _ffn, _i64, _p, _p, _p, _p, _p, _p, _p,
               _size, _p]),
    "bux_mx_pack_rows": (_int, [_p, _p, _i32, _i64, _i64, _i64, _p, _p]),
    "bux_mx_unpack_rows": (_int, [_p, _i64, _i64, _p, _p]),
    "bux_route_workspace_size": (_size, [_i64, _i32]),
    "bux_route": (
        _int, [_p, _p, _p, _i64, _i64, _i32, _f32, _int, _i32, _p, _i32, _i32, _i32, _int, _f32,
               _p, _p, _p, _p, _p, _p, _size, _p]),
}

# Constants of include/bux_amd.h.
MX_ROWS, MX_COLUMNS, MX_TILES, MX_HALVES = 1, 2, 4, 8
BF16, F32 = 0, 1
# the activations, bux_ffn.activation
ACTIVATIONS = {"swish": 0, "quick_gelu": 1, "relu": 2, "relu2": 3, "gelu": 4, "gelu_tanh": 5,
               "sigmoid": 6, "tanh": 7, "softplus": 8, "situ": 9}
NOALLOC_SCRATCH_BYTES = 262144
LIST_MAGIC, LIST_REFUSED = 0x54585542, 1
LAYERNORM, RMSNORM = 0, 1
ROUTER_SOFTMAX, ROUTER_SIGMOID, ROUTER_SQRTSOFTPLUS = 0, 1, 2


class BuxError(RuntimeError):
    """A call into the library failed: its code and message."""


_LIB = None


def load(path: str = PATH) -> ctypes.CDLL:
    """Return the library, loaded once, each entry point typed. Raises if it is not
    built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise BuxError(f"{path} is not built: run `python -m bux_amd.build`")
    lib = ctypes.CDLL(path)
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _LIB = lib
    return lib


def check(rc: int) -> None:
    """Raise `BuxError` with the library's message if `rc` is nonzero."""
    if rc != 0:
        msg = load().bux_last_error().decode(errors="replace")
        raise BuxError(f"bux_amd error {rc}: {msg}")
