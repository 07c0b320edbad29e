"""The C-ABI without a GPU: the built library loads, exports every entry point that
include/bux_amd.h declares (and the ctypes table types each of them), and its host-side
checks turn bad shapes, flags and workspaces into error codes and messages before any
kernel launch."""

import ctypes
import os
import re

import pytest

from bux_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "bux_amd.h")


def _declared() -> set[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(bux_\w+)\s*\(", text))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.PATH):
        pytest.fail(f"{_lib.PATH} is not built: run python -m bux_amd.build")
    return _lib.load()


def test_every_declared_entry_point_is_exported_and_typed(lib):
    declared = _declared()
    assert len(declared) >= 15
    assert declared == set(_lib.SIGNATURES), declared ^ set(_lib.SIGNATURES)
    for name in declared:
        assert hasattr(lib, name), name


def test_version(lib):
    assert lib.bux_version() >= 100


def test_workspace_sizes(lib):
    # counts of each bin in each segment of 256 picks, then the bins' totals and bases
    assert lib.bux_moe_permute_workspace_size(131072, 128) == (512 + 2) * 129 * 4
    assert lib.bux_moe_permute_workspace_size(0, 8) == 2 * 9 * 4
    # group starts, then a tile list: tiles of 256 rows, one more a group at most
    assert lib.bux_mx_grouped_rows_workspace_size(128, 131072, 131072) >= (512 + 128) * 12
    # a list of the group starts alone: a 64-byte header, then groups + 2 starts
    assert lib.bux_mx_grouped_contract_workspace_size(128) == 768


def _msg(lib) -> str:
    return lib.bux_last_error().decode()


def test_quantize_rejects_bad_shapes_and_flags(lib):
    p = ctypes.c_void_p(16)  # never dereferenced: the checks fail first
    rc = lib.bux_mx_quantize(p, None, 1, 64, 1, 64, 48, 64, None, 3, p, p, p, p, None)
    assert rc == 1 and "cols=48" in _msg(lib)
    rc = lib.bux_mx_quantize(p, None, 1, 64, 1, 64, 64, 40, None, 3, p, p, p, p, None)
    assert rc == 1 and "height=40" in _msg(lib)
    rc = lib.bux_mx_quantize(p, None, 1, 64, 1, 64, 64, 64, None, 0, p, p, p, p, None)
    assert rc == 1 and "flags" in _msg(lib)
    rc = lib.bux_mx_quantize(p, None, 1, 64, 1, 64, 64, 64, None, 4, p, p, p, p, None)
    assert rc == 1 and "flags=4" in _msg(lib)  # tiles alone: no copy asked for
    rc = lib.bux_mx_quantize(p, None, 1, 64, 1, 64, 64, 64, None, 16 | 1, p, p, p, p, None)
    assert rc == 1 and "flags=17" in _msg(lib)
    rc = lib.bux_mx_quantize(p, None, 1, 64, 1, 64, 96, 64, None, 8 | 1, p, p, p, p, None)
    assert rc == 1 and "BUX_MX_HALVES" in _msg(lib)  # halves: whole 64s of columns
    rc = lib.bux_mx_quantize(p, None, 1, 64, 1, 64, 64, 64, None, 2, p, p, None, None, None)
    assert rc == 1 and "t_values" in _msg(lib)
    rc = lib.bux_mx_quantize(p, p, 1, 64, 2, 64, 64, 64, None, 1, p, p, None, None, None)
    assert rc == 1 and "index" in _msg(lib)
    rc = lib.bux_mx_quantize(p, p, 0, 64, 1, 64, 64, 64, None, 1, p, p, None, None, None)
    assert rc == 1 and "index_div" in _msg(lib)
    rc = lib.bux_mx_quantize(p, p, 1, -1, 1, 64, 64, 64, None, 1, p, p, None, None, None)
    assert rc == 1 and "sources=-1" in _msg(lib)


def test_gemms_reject_bad_shapes_and_small_workspaces(lib):
    p = ctypes.c_void_p(16)
    rc = lib.bux_mx_grouped_rows(p, p, p, p, p, 4, 128, 128, 100, 128, 0, p, p, 1 << 20, None)
    assert rc == 1 and "k=100" in _msg(lib)
    # the tiled layout's K is whole 128s
    rc = lib.bux_mx_grouped_rows(p, p, p, p, p, 4, 128, 128, 160, 128, 0, p, p, 1 << 20, None)
    assert rc == 1 and "k=160" in _msg(lib)
    rc = lib.bux_mx_grouped_rows(p, p, p, p, p, 4, 128, 128, 128, 128, 0, p, p, 8, None)
    assert rc == 2 and "workspace" in _msg(lib)
    rc = lib.bux_mx_grouped_rows(p, p, p, p, p, 0, 128, 128, 128, 128, 0, p, p, 1 << 20, None)
    assert rc == 1 and "groups=0" in _msg(lib)
    rc = lib.bux_mx_grouped_rows(p, p, p, p, p, 4, 128, 128, 128, 128, 7, p, p, 1 << 20, None)
    assert rc == 1 and "out_dtype" in _msg(lib)
    rc = lib.bux_mx_grouped_contract(p, p, p, p, p, 4, 64, 64, 100, 0, p, p, 1 << 10, None)
    assert rc == 1 and "m=100" in _msg(lib)
    # an operand's bytes have no cap, its rows do (a K chunk's rows x 64 bytes in 2 GiB)
    rows = 33_554_177
    rc = lib.bux_mx_grouped_rows(p, p, p, p, p, 4, rows, 128, 128, rows, 0, p, p, 1 << 40, None)
    assert rc == 1 and "rows exceeds 33554176" in _msg(lib)
    rc = lib.bux_mx_grouped_contract(p, p, p, p, p, 4, rows, 64, 128, 0, p, p, 1 << 10, None)
    assert rc == 1 and "rows exceeds 33554176" in _msg(lib)
    rc = lib.bux_mx_grouped_contract(p, p, p, p, p, 4, 64, 64, 128, 0, p, p, 4, None)
    assert rc == 2 and "workspace" in _msg(lib)
    # any n and k (off multiples of 8 and past 2 GiB: the any-shape kernels); rows in int32
    rc = lib.bux_bf16_grouped_rows(p, p, 0, p, 4, 64, 100, 37, p, p, 8, None)
    assert rc == 2 and "workspace" in _msg(lib)
    rc = lib.bux_bf16_grouped_rows(p, p, 0, p, 4, 64, 128, 64, p, p, 8, None)
    assert rc == 2 and "workspace" in _msg(lib)
    assert lib.bux_bf16_grouped_rows_workspace_size(4, 64) >= 64 + 6 * 4 + 6 * 12
    rc = lib.bux_bf16_grouped_rows(p, p, 1, p, 4, 1 << 31, 128, 2048, p, p, 1 << 30, None)
    assert rc == 1 and "m=2147483648 rows" in _msg(lib)
    rc = lib.bux_bf16_grouped_contract(p, p, p, 4, 64, 45, 100, p, p, 4, None)
    assert rc == 2 and "workspace" in _msg(lib)
    rc = lib.bux_bf16_grouped_contract(p, p, p, 4, 1 << 31, 64, 128, p, p, 1 << 10, None)
    assert rc == 1 and "m=2147483648 rows" in _msg(lib)


def test_fused_up_gemm_rejects_bad_arguments(lib):
    p = ctypes.c_void_p(16)
    ws = lib.bux_mx_grouped_glu_workspace_size(4, 256)
    # group starts, then tiles of 256 rows with up to 31 more a group, one more a group
    assert ws >= (-(-(256 + 32 * 5) // 256) + 5) * 12

    def glu(height=256, n=128, k=128, rows=200, act=0, ws_bytes=1 << 20, groups=4, gated=1):
        ffn = _lib.FfnStruct(act, gated, 0, 0.0, 0, 0.0, 0.0)
        return lib.bux_mx_grouped_glu(p, p, p, p, p, groups, height, n, k, rows, p,
                                      ctypes.byref(ffn), p, p, p, p, p, p, ws_bytes, None)

    assert glu(height=200) == 1 and "height=200" in _msg(lib)  # whole 128s: h^T's K
    assert glu(n=96) == 1 and "n=96" in _msg(lib)  # (up, gate) pairs of f, a multiple of 32
    assert glu(k=64) == 1 and "k=64" in _msg(lib)
    assert glu(rows=300) == 1 and "rows=300" in _msg(lib)  # the product within the copies
    assert glu(act=5) == 1 and "activation 5" in _msg(lib)  # no fused gelu_tanh epilogue
    assert glu(act=0, gated=0) == 1 and "plain" in _msg(lib)
    assert glu(act=10) == 1 and "activation 10" in _msg(lib)
    assert glu(groups=0) == 1 and "groups=0" in _msg(lib)
    assert glu(ws_bytes=8) == 2 and "workspace" in _msg(lib)


def test_fused_dgrad_rejects_bad_arguments(lib):
    p = ctypes.c_void_p(16)
    ws = lib.bux_mx_grouped_dglu_workspace_size(4, 256, 200, 64)
    # the tile list, a float a row and 64 columns of d projected, 32 rows of d projected
    # a group (and the groups' end)
    assert ws >= 200 * 2 * 4 + 5 * 32 * 128 * 2

    def dglu(height=256, f=64, k=128, rows=200, act=0, ws_bytes=1 << 20, groups=4, gated=1):
        ffn = _lib.FfnStruct(act, gated, 0, 0.0, 0, 0.0, 0.0)
        return lib.bux_mx_grouped_dglu(p, p, p, p, p, groups, height, f, k, rows, p, p,
                                       ctypes.byref(ffn), None, p, p, p, p, p, p, ws_bytes, None)

    assert dglu(height=200) == 1 and "height=200" in _msg(lib)
    assert dglu(f=48) == 1 and "f=48" in _msg(lib)
    assert dglu(k=64) == 1 and "k=64" in _msg(lib)
    assert dglu(rows=300) == 1 and "rows=300" in _msg(lib)
    assert dglu(act=5) == 1 and "activation 5" in _msg(lib)
    assert dglu(act=0, gated=0) == 1 and "plain" in _msg(lib)
    assert dglu(groups=0) == 1 and "groups=0" in _msg(lib)
    assert dglu(ws_bytes=8) == 2 and "workspace" in _msg(lib)


def test_permute_and_token_ops_reject_bad_arguments(lib):
    p = ctypes.c_void_p(16)
    rc = lib.bux_moe_permute(p, 100, 0, p, p, p, p, p, 1 << 20, None)
    assert rc == 1 and "num_experts=0" in _msg(lib)
    rc = lib.bux_moe_permute(p, 1000, 8, p, p, p, p, p, 4, None)
    assert rc == 2 and "workspace" in _msg(lib)
    rc = lib.bux_token_sums(p, 10, p, 5, 2, 12, p, None)
    assert rc == 1 and "width=12" in _msg(lib)
    ok = _lib.FfnStruct(0, 1, 0, 0.0, 0, 0.0, 0.0)
    rc = lib.bux_glu_forward(p, p, None, 10, 6, ctypes.byref(ok), p, None)
    assert rc == 1 and "f=6" in _msg(lib)
    for bad, words in (((10, 1, 0, 0.0, 0, 0.0, 0.0), "activation 10"),
                       ((-1, 1, 0, 0.0, 0, 0.0, 0.0), "activation -1"),
                       ((0, 1, 1, -1.0, 0, 0.0, 0.0), "limit -1"),
                       ((0, 1, 1, float("nan"), 0, 0.0, 0.0), "limit nan"),
                       ((0, 0, 0, 0.0, 1, 0.0, 0.0), "up_softcap 0"),
                       ((0, 0, 0, 0.0, 1, -2.0, 0.0), "up_softcap -2")):
        ffn = _lib.FfnStruct(*bad)
        rc = lib.bux_glu_forward(p, p, None, 10, 8, ctypes.byref(ffn), p, None)
        assert rc == 1 and words in _msg(lib), (bad, _msg(lib))
        rc = lib.bux_glu_backward_quantize(p, p, p, None, 10, 32, ctypes.byref(ffn), 128, None, p, p,
                                           p, p, p, p, 1 << 20, None)
        assert rc == 1 and words in _msg(lib), (bad, _msg(lib))
    rc = lib.bux_glu_forward(p, p, None, 10, 8, None, p, None)
    assert rc == 1 and "NULL ffn" in _msg(lib)
    # a clamp at 0 clips every up to 0: allowed
    zero = _lib.FfnStruct(0, 1, 1, 0.0, 0, 0.0, 0.0)
    assert lib.bux_glu_forward(p, p, None, 0, 8, ctypes.byref(zero), p, None) == 0


def test_bias_ops_reject_bad_arguments(lib):
    p = ctypes.c_void_p(16)
    rc = lib.bux_expert_bias_add(p, 10, 12, p, p, 4, None)
    assert rc == 1 and "width=12" in _msg(lib)
    rc = lib.bux_expert_bias_add(p, 10, 16, p, None, 4, None)
    assert rc == 1 and "offsets" in _msg(lib)
    rc = lib.bux_expert_bias_add(p, 10, 16, p, p, 0, None)
    assert rc == 1 and "0 experts" in _msg(lib)
    assert lib.bux_expert_bias_add(None, 0, 16, None, p, 4, None) == 0  # no rows
    rc = lib.bux_expert_sums(p, p, 0, 10, None, 10, 16, p, 4, p, None)
    assert rc == 1 and "index_div=0" in _msg(lib)
    rc = lib.bux_expert_sums(p, p, 1, -1, None, 10, 16, p, 4, p, None)
    assert rc == 1 and "sources=-1" in _msg(lib)
    rc = lib.bux_expert_sums(p, None, 1, 0, None, 10, 16, p, 4, None, None)
    assert rc == 1 and "NULL" in _msg(lib)
    rc = lib.bux_token_sums_biased(p, 10, p, 5, 2, 16, None, p, 4, p, p, None)
    assert rc == 1 and "NULL bias" in _msg(lib)
    rc = lib.bux_token_sums_biased(p, 10, p, 5, 2, 12, p, p, 4, p, p, None)
    assert rc == 1 and "width=12" in _msg(lib)
    rc = lib.bux_expert_bias_weight_grad(p, p, 0, 10, 10, 16, p, p, 4, p, None)
    assert rc == 1 and "index_div=0" in _msg(lib)
    rc = lib.bux_expert_bias_weight_grad(p, p, 1, -1, 10, 16, p, p, 4, p, None)
    assert rc == 1 and "sources=-1" in _msg(lib)
    rc = lib.bux_expert_bias_weight_grad(p, None, 1, 0, 10, 16, p, p, 0, p, None)
    assert rc == 1 and "0 experts" in _msg(lib)


def test_float32_twins_reject_what_their_bfloat16_twins_reject(lib):
    """Each float32 twin checks its arguments as its bfloat16 twin does, before any
    launch, and names itself in the error."""
    p = ctypes.c_void_p(16)
    norm = _lib.NormStruct(_lib.RMSNORM, 1, 0, 0, 0, 1e-6)
    ffn = _lib.FfnStruct(0, 1, 0, 0.0, 0, 0.0, 0.0)
    cases = [
        ("bux_expert_bias_add", (p, 10, 12, p, p, 4, None), 1, "width=12"),
        ("bux_expert_sums", (p, p, 0, 10, None, 10, 16, p, 4, p, None), 1, "index_div=0"),
        ("bux_token_sums_biased", (p, 10, p, 5, 2, 16, None, p, 4, p, p, None), 1, "NULL bias"),
        ("bux_expert_bias_weight_grad", (p, p, 1, -1, 10, 16, p, p, 4, p, None), 1, "sources=-1"),
        ("bux_expert_norm_forward", (p, 10, 12, None, p, 4, ctypes.byref(norm), p, None, p, p, None),
         1, "d=12"),
        ("bux_expert_norm_backward", (p, None, 1, 0, p, 10, 16, None, p, 4, ctypes.byref(norm), p, None,
                                      p, p, p, p, None, p, 4, None), 2, "workspace"),
        ("bux_glu_forward", (p, p, None, 10, 6, ctypes.byref(ffn), p, None), 1, "f=6"),
        ("bux_glu_backward", (p, p, p, None, 10, 6, ctypes.byref(ffn), p, p, None), 1, "f=6"),
        ("bux_bf16_grouped_rows", (p, p, 0, p, 4, 64, 100, 37, p, p, 8, None), 2, "workspace"),
        ("bux_bf16_grouped_rows", (p, p, 1, p, 4, 1 << 31, 128, 2048, p, p, 1 << 30, None), 1,
         "m=2147483648 rows"),
        ("bux_bf16_grouped_contract", (p, p, p, 0, 64, 45, 100, p, p, 1 << 10, None), 1, "groups=0"),
    ]
    for name, args, code, text in cases:
        for twin in (name, name + "_f32"):
            rc = getattr(lib, twin)(*args)
            assert rc == code and text in _msg(lib) and twin in _msg(lib), (twin, rc, _msg(lib))


def test_route_rejects_bad_arguments(lib):
    p = ctypes.c_void_p(16)
    f = ctypes.c_float

    def route(t=8, d=64, n=16, router=0, scored=16, groups=1, keep=1, k=4, ws=1 << 20, sinks=None):
        return lib.bux_route(p, p, None, t, d, n, f(1.0), router, scored, None, groups, keep, k,
                             1, f(1.0), p, p, sinks, None, None, p, ws, None)

    assert lib.bux_route_workspace_size(2048, 128) == 128 * 2048 * 2
    assert lib.bux_route_workspace_size(64, 20) == 32 * 64 * 2  # experts padded to 32
    assert route(d=40) == 1 and "d=40" in _msg(lib)
    assert route(n=1025, scored=1025) == 1 and "n_logits=1025" in _msg(lib)
    assert route(k=17) == 1 and "k=17" in _msg(lib)
    assert route(router=3) == 1 and "router=3" in _msg(lib)
    assert route(groups=3) == 1 and "groups=3" in _msg(lib)
    assert route(groups=4, keep=5) == 1 and "keep=5" in _msg(lib)
    assert route(groups=8, keep=1, k=4) == 1 and "fewer than k=4" in _msg(lib)
    assert route(n=18, scored=16) == 1 and "NULL" in _msg(lib)  # sinks, none given
    assert route(t=0, n=18, scored=16) == 0  # no tokens: nothing to write
    assert route(ws=16) == 2 and "workspace" in _msg(lib)


def test_wire_rows_reject_bad_arguments(lib):
    p = ctypes.c_void_p(16)
    rc = lib.bux_mx_pack_rows(p, None, 1, 10, 10, 48, p, None)
    assert rc == 1 and "d=48" in _msg(lib)
    rc = lib.bux_mx_pack_rows(p, None, 1, 10, 11, 64, p, None)
    assert rc == 1 and "without an index" in _msg(lib)
    rc = lib.bux_mx_pack_rows(p, p, 0, 10, 20, 64, p, None)
    assert rc == 1 and "index_div=0" in _msg(lib)
    assert lib.bux_mx_pack_rows(None, None, 1, 0, 0, 64, None, None) == 0  # nothing to pack
    rc = lib.bux_mx_unpack_rows(p, 10, 40, p, None)
    assert rc == 1 and "d=40" in _msg(lib)
    rc = lib.bux_mx_unpack_rows(None, 10, 64, p, None)
    assert rc == 1 and "NULL" in _msg(lib)


def test_a_missing_library_fails_loudly(tmp_path, monkeypatch):
    monkeypatch.setattr(_lib, "_LIB", None)
    with pytest.raises(_lib.BuxError, match="not built"):
        _lib.load(str(tmp_path / "libbux_amd.so"))


def test_tile_lists_reject_bad_arguments(lib):
    p = ctypes.c_void_p(16)
    need = lib.bux_mx_grouped_rows_workspace_size(4, 256, 200)
    assert lib.bux_mx_grouped_tiles(p, 4, 256, 200, p, need - 1, None) == 2
    assert "list of" in _msg(lib)
    assert lib.bux_mx_grouped_tiles(None, 4, 256, 200, p, need, None) == 1
    assert lib.bux_mx_grouped_tiles(p, 0, 256, 200, p, need, None) == 1 and "groups=0" in _msg(lib)
    rc = lib.bux_mx_grouped_rows_listed(p, p, p, p, None, need, 4, 256, 128, 128, 200, 0, p, None)
    assert rc == 1 and "NULL list" in _msg(lib)
    rc = lib.bux_mx_grouped_rows_listed(p, p, p, p, p, need, 4, 256, 128, 100, 200, 0, p, None)
    assert rc == 1 and "k=100" in _msg(lib)
    # a list too short for the dimensions asked: refused before any launch
    rc = lib.bux_mx_grouped_rows_listed(p, p, p, p, p, need, 4, 256, 128, 128, 4096, 0, p, None)
    assert rc == 2 and "height=4096" in _msg(lib)
    rc = lib.bux_mx_grouped_rows_listed(p, p, p, p, p, need, 64, 256, 128, 128, 200, 0, p, None)
    assert rc == 2 and "groups=64" in _msg(lib)
    rc = lib.bux_mx_grouped_contract_listed(p, p, p, p, p, need, 4, 64, 64, 100, 0, p, None)
    assert rc == 1 and "m=100" in _msg(lib)
    rc = lib.bux_mx_grouped_contract_listed(p, p, p, p, p, 16, 4, 64, 64, 128, 0, p, None)
    assert rc == 2 and "16 bytes" in _msg(lib)


def test_every_entry_point_has_an_xla_ffi_handler():
    """bux_amd/xla/xla_ffi.cc binds every compute entry point for jax.ffi (the workspace
    sizes are trace-time queries through ctypes; the entry point that allocates nothing
    is for callers outside XLA, which owns every buffer). A float32 twin is called from
    its bfloat16 twin's handler, which picks by the buffer's element type."""
    src = open(os.path.join(ROOT, "bux_amd", "xla", "xla_ffi.cc")).read()
    called = set(re.findall(r"\b(bux_\w+)\(", src)) - {"bux_last_error"}
    wanted = {n for n in _declared()
              if not n.endswith("_workspace_size")
              and n not in ("bux_last_error", "bux_version", "bux_mx_grouped_rows_noalloc")}
    assert wanted <= called, wanted - called
    twins = {n for n in wanted if n.endswith("_f32")}
    assert {n[:-4] for n in twins} <= wanted
    handlers = len(re.findall(r"XLA_FFI_DEFINE_HANDLER_SYMBOL\(", src))
    assert handlers == len(wanted - twins)


def _calls(text: str, name_re: str) -> dict[str, list[int]]:
    """Each `name(` in text: the number of its top-level arguments (commas outside
    nested parentheses, brackets and angle-bracketed template arguments)."""
    found: dict[str, list[int]] = {}
    for m in re.finditer(name_re, text):
        i, depth, args, saw = m.end(), 1, 0, False
        while depth:
            c = text[i]
            if c in "([{<":
                depth += 1
            elif c in ")]}>":
                depth -= 1
            elif c == "," and depth == 1:
                args += 1
            elif not c.isspace():
                saw = True
            i += 1
        found.setdefault(m.group(1), []).append(args + 1 if saw else 0)
    return found


def test_each_xla_ffi_handler_passes_every_argument_the_header_declares():
    """xla_ffi.cc compiles only where the XLA FFI headers are: the argument count of each
    of its calls into the library must match the declaration in include/bux_amd.h."""
    header = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    declared = {n: counts[0] for n, counts in
                _calls(header, r"\b(?:int|size_t|const char\*)\s+(bux_\w+)\s*\(").items()}
    src = open(os.path.join(ROOT, "bux_amd", "xla", "xla_ffi.cc")).read()
    src = re.sub(r"//[^\n]*", "", src).replace("->", ".")
    calls = _calls(src, r"\b(bux_\w+)\(")
    calls.pop("bux_last_error", None)
    assert calls
    for name, counts in calls.items():
        assert name in declared, name
        assert set(counts) == {declared[name]}, (name, counts, declared[name])
