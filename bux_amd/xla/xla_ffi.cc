// XLA FFI handlers for every entry point of libbux_amd (include/bux_amd.h): what bux
// binds as jax.ffi targets so that the kernels run inside jit on XLA's stream, with XLA
// owning every buffer. Each handler unpacks XLA's buffers, reads the shapes the C ABI
// takes from them, calls the entry point on XLA's stream and turns a nonzero status into
// an ffi::Error carrying bux_last_error().
//
// Conventions: an empty buffer (0 bytes) stands for a NULL argument (an absent index,
// `filled`, bias, copy not asked for); settings are attributes; in-place outputs
// (bux_expert_bias_add's x, bux_expert_bias_weight_grad's d_weights) are results the
// caller aliases to their input (jax.ffi.ffi_call's input_output_aliases). A listed
// GEMM's tile list is an argument: the kernels write it only to refuse a list made for
// other dimensions.
//
// Built only where the XLA FFI headers are (jax.ffi.include_dir(), or
// BUX_XLA_FFI_INCLUDE): `python -m bux_amd.build` makes libbux_amd_xla.so next to
// libbux_amd.so then, and skips it otherwise. Without the headers this file is empty.

#if __has_include("xla/ffi/api/ffi.h")

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "bux_amd.h"
#include "xla/ffi/api/ffi.h"

namespace ffi = xla::ffi;

namespace {

using Stream = ffi::PlatformStream<hipStream_t>;
using In = ffi::AnyBuffer;
using Out = ffi::Result<ffi::AnyBuffer>;

template <typename T>
T* at(const In& b) {
  return b.size_bytes() ? static_cast<T*>(b.untyped_data()) : nullptr;
}
template <typename T>
T* at(Out& b) {
  return b->size_bytes() ? static_cast<T*>(b->untyped_data()) : nullptr;
}
int64_t dim(const In& b, int i) {
  const auto d = b.dimensions();
  return d[i < 0 ? static_cast<int>(d.size()) + i : i];
}
int64_t dim(Out& b, int i) {
  const auto d = b->dimensions();
  return d[i < 0 ? static_cast<int>(d.size()) + i : i];
}
ffi::Error status(int rc) {
  if (rc == 0) return ffi::Error::Success();
  return ffi::Error(ffi::ErrorCode::kInternal, std::string(bux_last_error()));
}
int dtype_of(Out& y) { return y->element_type() == ffi::DataType::F32 ? BUX_F32 : BUX_BF16; }
bool f32(const In& b) { return b.element_type() == ffi::DataType::F32; }

bux_ffn ffn_of(int64_t activation, int64_t gated, int64_t clamped, float limit, int64_t capped,
               float up_softcap, float up_offset) {
  return bux_ffn{static_cast<int32_t>(activation), static_cast<int32_t>(gated),
                 static_cast<int32_t>(clamped), limit, static_cast<int32_t>(capped), up_softcap,
                 up_offset};
}

bux_norm norm_of(int64_t kind, int64_t affine, int64_t zero_centered, int64_t scale_input,
                 int64_t bias, float eps) {
  return bux_norm{static_cast<int32_t>(kind), static_cast<int32_t>(affine),
                  static_cast<int32_t>(zero_centered), static_cast<int32_t>(scale_input),
                  static_cast<int32_t>(bias), eps};
}

}  // namespace

// The activation's settings (bux_ffn), as attributes.
#define BUX_FFN_ATTRS                                                                      \
  .Attr<int64_t>("activation").Attr<int64_t>("gated").Attr<int64_t>("clamped")            \
      .Attr<float>("limit").Attr<int64_t>("capped").Attr<float>("up_softcap")              \
      .Attr<float>("up_offset")
#define BUX_FFN_PARAMS                                                                     \
  int64_t activation, int64_t gated, int64_t clamped, float limit, int64_t capped,        \
      float up_softcap, float up_offset
#define BUX_FFN ffn_of(activation, gated, clamped, limit, capped, up_softcap, up_offset)
#define BUX_NORM_ATTRS                                                                     \
  .Attr<int64_t>("kind").Attr<int64_t>("affine").Attr<int64_t>("zero_centered")           \
      .Attr<int64_t>("scale_input").Attr<int64_t>("norm_bias").Attr<float>("eps")
#define BUX_NORM_PARAMS                                                                    \
  int64_t kind, int64_t affine, int64_t zero_centered, int64_t scale_input,               \
      int64_t norm_bias, float eps
#define BUX_NORM norm_of(kind, affine, zero_centered, scale_input, norm_bias, eps)

// --- a-1: the sort by expert ---------------------------------------------------------

static ffi::Error MoePermute(hipStream_t s, In idx, int64_t num_experts, Out order, Out inverse,
                             Out sizes, Out offsets, Out ws) {
  return status(bux_moe_permute(at<const int32_t>(idx), static_cast<int64_t>(idx.element_count()),
                                static_cast<int32_t>(num_experts), at<int32_t>(order),
                                at<int32_t>(inverse), at<int32_t>(sizes), at<int32_t>(offsets),
                                at<void>(ws), ws->size_bytes(), s));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(BuxMoePermute, MoePermute,
                              ffi::Ffi::Bind().Ctx<Stream>().Arg<In>().Attr<int64_t>("num_experts")
                                  .Ret<In>().Ret<In>().Ret<In>().Ret<In>().Ret<In>());

// --- a-4: MXFP8 quantization -----------------------------------------------------------

// x [groups, rows, cols] (or with an index the matrix read from), bfloat16 or float32;
// index and filled may be empty; a copy's results empty when not asked for.
static ffi::Error MxQuantize(hipStream_t s, In x, In index, In filled, int64_t index_div,
                             int64_t groups, int64_t rows, int64_t height, int64_t flags,
                             Out values, Out scales, Out t_values, Out t_scales) {
  if (f32(x))
    return status(bux_mx_quantize_f32(at<const float>(x), at<const int32_t>(index),
                                      static_cast<int32_t>(index_div), dim(x, 0), groups, rows,
                                      dim(x, -1), height, at<const int32_t>(filled),
                                      static_cast<int>(flags), at<uint8_t>(values),
                                      at<uint8_t>(scales), at<uint8_t>(t_values),
                                      at<uint8_t>(t_scales), s));
  return status(bux_mx_quantize(at<const uint16_t>(x), at<const int32_t>(index),
                                static_cast<int32_t>(index_div), dim(x, 0), groups, rows,
                                dim(x, -1), height,
                                at<const int32_t>(filled), static_cast<int>(flags),
                                at<uint8_t>(values), at<uint8_t>(scales), at<uint8_t>(t_values),
                                at<uint8_t>(t_scales), s));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(BuxMxQuantize, MxQuantize,
                              ffi::Ffi::Bind().Ctx<Stream>().Arg<In>().Arg<In>().Arg<In>()
                                  .Attr<int64_t>("index_div").Attr<int64_t>("groups")
                                  .Attr<int64_t>("rows").Attr<int64_t>("height")
                                  .Attr<int64_t>("flags")
                                  .Ret<In>().Ret<In>().Ret<In>().Ret<In>());

// --- a-6, a-7: the grouped MXFP8 GEMMs -----------------------------------------------------
// Tiled operands: a values [K/64, m, 64]; b values [g, K/64, n, 64]; the contract's a
// [M/64, d, 64] and b [M/64, f, 64].

static ffi::Error MxRows(hipStream_t s, In av, In as, In bv, In bs, In sizes, Out y, Out ws) {
  return status(bux_mx_grouped_rows(at<const uint8_t>(av), at<const uint8_t>(as),
                                    at<const uint8_t>(bv), at<const uint8_t>(bs),
                                    at<const int32_t>(sizes), static_cast<int32_t>(dim(bv, 0)),
                                    dim(av, 1), dim(bv, 2), dim(av, 0) * 64, dim(y, 0),
                                    dtype_of(y), at<void>(y), at<void>(ws), ws->size_bytes(), s));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(BuxMxRows, MxRows,
                              ffi::Ffi::Bind().Ctx<Stream>().Arg<In>().Arg<In>().Arg<In>()
                                  .Arg<In>().Arg<In>().Ret<In>().Ret<In>());

static ffi::Error MxRowsStarted(hipStream_t s, In av, In as, In bv, In bs, In sizes, In starts,
                                Out y, Out ws) {
  return status(bux_mx_grouped_rows_started(
      at<const uint8_t>(av), at<const uint8_t>(as), at<const uint8_t>(bv), at<const uint8_t>(bs),
      at<const int32_t>(sizes), at<const int32_t>(starts), static_cast<int32_t>(dim(bv, 0)),
      dim(av, 1), dim(bv, 2), dim(av, 0) * 64, dim(y, 0), dtype_of(y), at<void>(y),
      at<void>(ws), ws->size_bytes(), s));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(BuxMxRowsStarted, MxRowsStarted,
                              ffi::Ffi::Bind().Ctx<Stream>().Arg<In>().Arg<In>().Arg<In>()
                                  .Arg<In>().Arg<In>().Arg<In>().Ret<In>().Ret<In>());

static ffi::Error MxTiles(hipStream_t s, In sizes, int64_t m, int64_t height, Out list) {
  return status(bux_mx_grouped_tiles(at<const int32_t>(sizes),
                                     static_cast<int32_t>(sizes.element_count()), m, height,
                                     at<void>(list), list->size_bytes(), s));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(BuxMxTiles, MxTiles,
                              ffi::Ffi::Bind().Ctx<Stream>().Arg<In>().Attr<int64_t>("m")
                                  .Attr<int64_t>("height").Ret<In>());

static ffi::Error MxRowsListed(hipStream_t s, In av, In as, In bv, In bs, In list, Out y) {
  return status(bux_mx_grouped_rows_listed(
      at<const uint8_t>(av), at<const uint8_t>(as), at<const uint8_t>(bv), at<const uint8_t>(bs),
      at<void>(list), list.size_bytes(), static_cast<int32_t>(dim(bv, 0)), dim(av, 1), dim(bv, 2),
      dim(av, 0) * 64, dim(y, 0), dtype_of(y), at<void>(y), s));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(BuxMxRowsListed, MxRowsListed,
                              ffi::Ffi::Bind().Ctx<Stream>().Arg<In>().Arg<In>().Arg<In>()
                                  .Arg<In>().Arg<In>().Ret<In>());

static ffi::Error MxContract(hipStream_t s, In av, In as, In bv, In bs, In sizes, Out dw,
                             Out ws) {
  return status(bux_mx_grouped_contract(
      at<const uint8_t>(av), at<const uint8_t>(as), at<const uint8_t>(bv), at<const uint8_t>(bs),
      at<const int32_t>(sizes), static_cast<int32_t>(sizes.element_count()), dim(av, 1),
      dim(bv, 1), dim(av, 0) * 64, dtype_of(dw), at<void>(dw), at<void>(ws), ws->size_bytes(),
      s));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(BuxMxContract, MxContract,
                              ffi::Ffi::Bind().Ctx<Stream>().Arg<In>().Arg<In>().Arg<In>()
                                  .Arg<In>().Arg<In>().Ret<In>().Ret<In>());

static ffi::Error MxContractListed(hipStream_t s, In av, In as, In bv, In bs, In list,
                                   int64_t groups, Out dw) {
  return status(bux_mx_grouped_contract_listed(
      at<const uint8_t>(av), at<const uint8_t>(as), at<const uint8_t>(bv), at<const uint8_t>(bs),
      at<void>(list), list.size_bytes(), static_cast<int32_t>(groups), dim(av, 1), dim(bv, 1),
      dim(av, 0) * 64, dtype_of(dw), at<void>(dw), s));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(BuxMxContractListed, MxContractListed,
                              ffi::Ffi::Bind().Ctx<Stream>().Arg<In>().Arg<In>().Arg<In>()
                                  .Arg<In>().Arg<In>().Attr<int64_t>("groups").Ret<In>());

// --- a-10: the bfloat16 grouped GEMMs ----------------------------------------------------

// ws: a u8 result of bux_bf16_grouped_rows_workspace_size (_contract_) bytes.
// float32 x (a layer in float32): bux_bf16_grouped_rows_f32 (_contract_f32), the same
// workspace.
static ffi::Error Bf16Rows(hipStream_t s, In x, In w, In sizes, int64_t transposed, Out y,
                           Out ws) {
  if (f32(x))
    return status(bux_bf16_grouped_rows_f32(at<const float>(x), at<const float>(w),
                                            static_cast<int>(transposed), at<const int32_t>(sizes),
                                            static_cast<int32_t>(dim(w, 0)), dim(x, 0), dim(y, 1),
                                            dim(x, 1), at<float>(y), at<void>(ws),
                                            ws->size_bytes(), s));
  return status(bux_bf16_grouped_rows(at<const uint16_t>(x), at<const uint16_t>(w),
                                      static_cast<int>(transposed), at<const int32_t>(sizes),
                                      static_cast<int32_t>(dim(w, 0)), dim(x, 0), dim(y, 1),
                                      dim(x, 1), at<uint16_t>(y), at<void>(ws), ws->size_bytes(),
                                      s));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(BuxBf16Rows, Bf16Rows,
                              ffi::Ffi::Bind().Ctx<Stream>().Arg<In>().Arg<In>().Arg<In>()
                                  .Attr<int64_t>("transposed").Ret<In>().Ret<In>());

static ffi::Error Bf16Contract(hipStream_t s, In x, In dy, In sizes, Out dw, Out ws) {
  if (f32(x))
    return status(bux_bf16_grouped_contract_f32(at<const float>(x), at<const float>(dy),
                                                at<const int32_t>(sizes),
                                                static_cast<int32_t>(sizes.element_count()),
                                                dim(x, 0), dim(x, 1), dim(dy, 1), at<float>(dw),
                                                at<void>(ws), ws->size_bytes(), s));
  return status(bux_bf16_grouped_contract(at<const uint16_t>(x), at<const uint16_t>(dy),
                                          at<const int32_t>(sizes),
                                          static_cast<int32_t>(sizes.element_count()), dim(x, 0),
                                          dim(x, 1), dim(dy, 1), at<uint16_t>(dw), at<void>(ws),
                                          ws->size_bytes(), s));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(BuxBf16Contract, Bf16Contract,
                              ffi::Ffi::Bind().Ctx<Stream>().Arg<In>().Arg<In>().Arg<In>()
                                  .Ret<In>().Ret<In>());

// --- a-2, a-3: the token path's gathers and sums ---------------------------------------

static ffi::Error TokenRows(hipStream_t s, In z, In order, int64_t k, Out rows) {
  return status(bux_token_rows(at<const uint16_t>(z), dim(z, 0), at<const int32_t>(order),
                               dim(rows, 0), static_cast<int32_t>(k), dim(z, -1),
                               at<uint16_t>(rows), s));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(BuxTokenRows, TokenRows,
                              ffi::Ffi::Bind().Ctx<Stream>().Arg<In>().Arg<In>()
                                  .Attr<int64_t>("k").Ret<In>());

// inverse [t, k]; y and out bfloat16 or float32
static ffi::Error TokenSums(hipStream_t s, In y, In inverse, Out out) {
  if (f32(y))
    return status(bux_token_sums_f32(at<const float>(y), dim(y, 0), at<const int32_t>(inverse),
                                     dim(inverse, 0), static_cast<int32_t>(dim(inverse, 1)),
                                     dim(y, 1), at<float>(out), s));
  return status(bux_token_sums(at<const uint16_t>(y), dim(y, 0), at<const int32_t>(inverse),
                               dim(inverse, 0), static_cast<int32_t>(dim(inverse, 1)), dim(y, 1),
                               at<uint16_t>(out), s));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(BuxTokenSums, TokenSums,
                              ffi::Ffi::Bind().Ctx<Stream>().Arg<In>().Arg<In>().Ret<In>());

// --- a-8: the expert FFN's activation, biases and output norm ------------------------
// projected (m, f, 2) gated or (m, f) plain, as `gated` says; filled may be empty.

static ffi::Error GluForward(hipStream_t s, In projected, In weights, In filled, BUX_FFN_PARAMS,
                             Out h) {
  const bux_ffn ffn = BUX_FFN;
  if (f32(projected))  // a layer in float32
    return status(bux_glu_forward_f32(at<const float>(projected), at<const float>(weights),
                                      at<const int32_t>(filled), dim(h, 0), dim(h, 1), &ffn,
                                      at<float>(h), s));
  return status(bux_glu_forward(at<const uint16_t>(projected), at<const uint16_t>(weights),
                                at<const int32_t>(filled), dim(h, 0), dim(h, 1), &ffn,
                                at<uint16_t>(h), s));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(BuxGluForward, GluForward,
                              ffi::Ffi::Bind().Ctx<Stream>().Arg<In>().Arg<In>().Arg<In>()
                                  BUX_FFN_ATTRS.Ret<In>());

static ffi::Error GluBackward(hipStream_t s, In projected, In weights, In dh, In filled,
                              BUX_FFN_PARAMS, Out d_projected, Out d_weights) {
  const bux_ffn ffn = BUX_FFN;
  if (f32(projected))  // a layer in float32
    return status(bux_glu_backward_f32(at<const float>(projected), at<const float>(weights),
                                       at<const float>(dh), at<const int32_t>(filled), dim(dh, 0),
                                       dim(dh, 1), &ffn, at<float>(d_projected),
                                       at<float>(d_weights), s));
  return status(bux_glu_backward(at<const uint16_t>(projected), at<const uint16_t>(weights),
                                 at<const uint16_t>(dh), at<const int32_t>(filled), dim(dh, 0),
                                 dim(dh, 1), &ffn, at<uint16_t>(d_projected),
                                 at<uint16_t>(d_weights), s));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(BuxGluBackward, GluBackward,
                              ffi::Ffi::Bind().Ctx<Stream>().Arg<In>().Arg<In>().Arg<In>()
                                  .Arg<In>() BUX_FFN_ATTRS.Ret<In>().Ret<In>());

// h may be an empty result (not kept); f from the row copy's K is not exact, so it is an
// attribute, as are m and height.
static ffi::Error GluQuantize(hipStream_t s, In projected, In weights, In filled, BUX_FFN_PARAMS,
                              int64_t m, int64_t f, int64_t height, Out h, Out values, Out scales,
                              Out t_values, Out t_scales) {
  const bux_ffn ffn = BUX_FFN;
  if (f32(projected))  // a layer in float32: projected, weights and h float32
    return status(bux_glu_quantize_f32(at<const float>(projected), at<const float>(weights),
                                       at<const int32_t>(filled), m, f, &ffn, height,
                                       at<float>(h), at<uint8_t>(values), at<uint8_t>(scales),
                                       at<uint8_t>(t_values), at<uint8_t>(t_scales), s));
  return status(bux_glu_quantize(at<const uint16_t>(projected), at<const uint16_t>(weights),
                                 at<const int32_t>(filled), m, f, &ffn, height, at<uint16_t>(h),
                                 at<uint8_t>(values), at<uint8_t>(scales), at<uint8_t>(t_values),
                                 at<uint8_t>(t_scales), s));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(BuxGluQuantize, GluQuantize,
                              ffi::Ffi::Bind().Ctx<Stream>().Arg<In>().Arg<In>().Arg<In>()
                                  BUX_FFN_ATTRS.Attr<int64_t>("m").Attr<int64_t>("f")
                                  .Attr<int64_t>("height").Ret<In>().Ret<In>().Ret<In>()
                                  .Ret<In>().Ret<In>());

static ffi::Error GluBackwardQuantize(hipStream_t s, In projected, In weights, In dh, In filled,
                                      BUX_FFN_PARAMS, int64_t height, Out d_projected,
                                      Out values, Out scales, Out t_values, Out t_scales,
                                      Out d_weights, Out ws) {
  const bux_ffn ffn = BUX_FFN;
  if (f32(projected))  // a layer in float32
    return status(bux_glu_backward_quantize_f32(
        at<const float>(projected), at<const float>(weights), at<const float>(dh),
        at<const int32_t>(filled), dim(dh, 0), dim(dh, 1), &ffn, height, at<float>(d_projected),
        at<uint8_t>(values), at<uint8_t>(scales), at<uint8_t>(t_values), at<uint8_t>(t_scales),
        at<float>(d_weights), at<void>(ws), ws->size_bytes(), s));
  return status(bux_glu_backward_quantize(
      at<const uint16_t>(projected), at<const uint16_t>(weights), at<const uint16_t>(dh),
      at<const int32_t>(filled), dim(dh, 0), dim(dh, 1), &ffn, height, at<uint16_t>(d_projected),
      at<uint8_t>(values), at<uint8_t>(scales), at<uint8_t>(t_values), at<uint8_t>(t_scales),
      at<uint16_t>(d_weights), at<void>(ws), ws->size_bytes(), s));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(BuxGluBackwardQuantize, GluBackwardQuantize,
                              ffi::Ffi::Bind().Ctx<Stream>().Arg<In>().Arg<In>().Arg<In>()
                                  .Arg<In>() BUX_FFN_ATTRS.Attr<int64_t>("height")
                                  .Ret<In>().Ret<In>().Ret<In>().Ret<In>().Ret<In>().Ret<In>()
                                  .Ret<In>());

static ffi::Error MxGroupedGlu(hipStream_t s, In av, In as, In bv, In bs, In sizes, In weights,
                               BUX_FFN_PARAMS, Out projected, Out values, Out scales,
                               Out t_values, Out t_scales, Out ws) {
  const bux_ffn ffn = BUX_FFN;
  return status(bux_mx_grouped_glu(
      at<const uint8_t>(av), at<const uint8_t>(as), at<const uint8_t>(bv), at<const uint8_t>(bs),
      at<const int32_t>(sizes), static_cast<int32_t>(dim(bv, 0)), dim(av, 1), dim(bv, 2),
      dim(av, 0) * 64, dim(projected, 0), at<const uint16_t>(weights), &ffn,
      at<uint16_t>(projected), at<uint8_t>(values), at<uint8_t>(scales), at<uint8_t>(t_values),
      at<uint8_t>(t_scales), at<void>(ws), ws->size_bytes(), s));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(BuxMxGroupedGlu, MxGroupedGlu,
                              ffi::Ffi::Bind().Ctx<Stream>().Arg<In>().Arg<In>().Arg<In>()
                                  .Arg<In>().Arg<In>().Arg<In>() BUX_FFN_ATTRS.Ret<In>()
                                  .Ret<In>().Ret<In>().Ret<In>().Ret<In>().Ret<In>());

// dy values [K/64, height, 64], W_down values [g, K/64, f, 64]; projected [rows, 2f]; the
// results d projected's two copies, then d_weights [rows], then the workspace.
static ffi::Error MxGroupedDglu(hipStream_t s, In av, In as, In bv, In bs, In sizes,
                                In projected, In weights, BUX_FFN_PARAMS, Out values,
                                Out scales, Out t_values, Out t_scales, Out d_weights, Out ws) {
  const bux_ffn ffn = BUX_FFN;
  return status(bux_mx_grouped_dglu(
      at<const uint8_t>(av), at<const uint8_t>(as), at<const uint8_t>(bv), at<const uint8_t>(bs),
      at<const int32_t>(sizes), static_cast<int32_t>(dim(bv, 0)), dim(av, 1), dim(bv, 2),
      dim(av, 0) * 64, dim(projected, 0), at<const uint16_t>(projected),
      at<const uint16_t>(weights), &ffn, nullptr, at<uint8_t>(values), at<uint8_t>(scales),
      at<uint8_t>(t_values), at<uint8_t>(t_scales), at<uint16_t>(d_weights), at<void>(ws),
      ws->size_bytes(), s));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(BuxMxGroupedDglu, MxGroupedDglu,
                              ffi::Ffi::Bind().Ctx<Stream>().Arg<In>().Arg<In>().Arg<In>()
                                  .Arg<In>().Arg<In>().Arg<In>().Arg<In>() BUX_FFN_ATTRS
                                  .Ret<In>().Ret<In>().Ret<In>().Ret<In>().Ret<In>().Ret<In>());

// The bias and norm entry points by element type: the bfloat16 ones (T uint16_t) or
// their float32 twins (T float); each handler picks by its rows' element type.
namespace {
int bias_add(uint16_t* x, int64_t m, int64_t w, const uint16_t* b, const int32_t* o, int32_t e,
             hipStream_t s) {
  return bux_expert_bias_add(x, m, w, b, o, e, s);
}
int bias_add(float* x, int64_t m, int64_t w, const float* b, const int32_t* o, int32_t e,
             hipStream_t s) {
  return bux_expert_bias_add_f32(x, m, w, b, o, e, s);
}
int expert_sums(const uint16_t* x, const int32_t* i, int32_t div, int64_t src,
                const uint16_t* w, int64_t m, int64_t width, const int32_t* o, int32_t e,
                float* out, hipStream_t s) {
  return bux_expert_sums(x, i, div, src, w, m, width, o, e, out, s);
}
int expert_sums(const float* x, const int32_t* i, int32_t div, int64_t src, const float* w,
                int64_t m, int64_t width, const int32_t* o, int32_t e, float* out,
                hipStream_t s) {
  return bux_expert_sums_f32(x, i, div, src, w, m, width, o, e, out, s);
}
int sums_biased(const uint16_t* y, int64_t rows, const int32_t* inv, int64_t t, int32_t k,
                int64_t width, const uint16_t* b, const int32_t* o, int32_t e,
                const uint16_t* w, uint16_t* out, hipStream_t s) {
  return bux_token_sums_biased(y, rows, inv, t, k, width, b, o, e, w, out, s);
}
int sums_biased(const float* y, int64_t rows, const int32_t* inv, int64_t t, int32_t k,
                int64_t width, const float* b, const int32_t* o, int32_t e, const float* w,
                float* out, hipStream_t s) {
  return bux_token_sums_biased_f32(y, rows, inv, t, k, width, b, o, e, w, out, s);
}
int weight_grad(const uint16_t* dy, const int32_t* i, int32_t div, int64_t src, int64_t m,
                int64_t width, const uint16_t* b, const int32_t* o, int32_t e, uint16_t* dw,
                hipStream_t s) {
  return bux_expert_bias_weight_grad(dy, i, div, src, m, width, b, o, e, dw, s);
}
int weight_grad(const float* dy, const int32_t* i, int32_t div, int64_t src, int64_t m,
                int64_t width, const float* b, const int32_t* o, int32_t e, float* dw,
                hipStream_t s) {
  return bux_expert_bias_weight_grad_f32(dy, i, div, src, m, width, b, o, e, dw, s);
}
int norm_forward(const uint16_t* y, int64_t m, int64_t d, const uint16_t* db, const int32_t* o,
                 int32_t e, const bux_norm* n, const uint16_t* sc, const uint16_t* b,
                 const uint16_t* w, uint16_t* out, hipStream_t s) {
  return bux_expert_norm_forward(y, m, d, db, o, e, n, sc, b, w, out, s);
}
int norm_forward(const float* y, int64_t m, int64_t d, const float* db, const int32_t* o,
                 int32_t e, const bux_norm* n, const float* sc, const float* b, const float* w,
                 float* out, hipStream_t s) {
  return bux_expert_norm_forward_f32(y, m, d, db, o, e, n, sc, b, w, out, s);
}
int norm_backward(const uint16_t* dy, const int32_t* i, int32_t div, int64_t src,
                  const uint16_t* y, int64_t m, int64_t d, const uint16_t* db, const int32_t* o,
                  int32_t e, const bux_norm* n, const uint16_t* sc, const uint16_t* b,
                  const uint16_t* w, uint16_t* dv, uint16_t* dw, float* dsc, float* dbias,
                  void* ws, size_t bytes, hipStream_t s) {
  return bux_expert_norm_backward(dy, i, div, src, y, m, d, db, o, e, n, sc, b, w, dv, dw, dsc,
                                  dbias, ws, bytes, s);
}
int norm_backward(const float* dy, const int32_t* i, int32_t div, int64_t src, const float* y,
                  int64_t m, int64_t d, const float* db, const int32_t* o, int32_t e,
                  const bux_norm* n, const float* sc, const float* b, const float* w, float* dv,
                  float* dw, float* dsc, float* dbias, void* ws, size_t bytes, hipStream_t s) {
  return bux_expert_norm_backward_f32(dy, i, div, src, y, m, d, db, o, e, n, sc, b, w, dv, dw,
                                      dsc, dbias, ws, bytes, s);
}
int32_t experts_in(const In& offsets) { return static_cast<int32_t>(offsets.element_count() - 1); }

template <typename T>
ffi::Error expert_bias_add_as(hipStream_t s, In bias, In offsets, Out& x_out) {
  return status(bias_add(at<T>(x_out), dim(x_out, 0),
                         static_cast<int64_t>(x_out->element_count()) / dim(x_out, 0),
                         at<const T>(bias), at<const int32_t>(offsets), experts_in(offsets), s));
}
template <typename T>
ffi::Error expert_sums_as(hipStream_t s, In x, In index, In weights, In offsets,
                          int64_t index_div, Out& out) {
  const int64_t m = index.size_bytes() ? static_cast<int64_t>(index.element_count()) : dim(x, 0);
  return status(expert_sums(at<const T>(x), at<const int32_t>(index),
                            static_cast<int32_t>(index_div), dim(x, 0), at<const T>(weights), m,
                            dim(out, 1), at<const int32_t>(offsets), experts_in(offsets),
                            at<float>(out), s));
}
template <typename T>
ffi::Error token_sums_biased_as(hipStream_t s, In y, In inverse, In bias, In offsets,
                                In weights, Out& out) {
  return status(sums_biased(at<const T>(y), dim(y, 0), at<const int32_t>(inverse),
                            dim(inverse, 0), static_cast<int32_t>(dim(inverse, 1)), dim(y, 1),
                            at<const T>(bias), at<const int32_t>(offsets), experts_in(offsets),
                            at<const T>(weights), at<T>(out), s));
}
template <typename T>
ffi::Error bias_weight_grad_as(hipStream_t s, In dy, In index, In bias, In offsets,
                               int64_t index_div, Out& d_weights_out) {
  return status(weight_grad(at<const T>(dy), at<const int32_t>(index),
                            static_cast<int32_t>(index_div), dim(dy, 0),
                            static_cast<int64_t>(d_weights_out->element_count()), dim(dy, 1),
                            at<const T>(bias), at<const int32_t>(offsets), experts_in(offsets),
                            at<T>(d_weights_out), s));
}
template <typename T>
ffi::Error norm_forward_as(hipStream_t s, In y, In down_bias, In offsets, In scale, In bias,
                           In weights, const bux_norm& norm, Out& out) {
  return status(norm_forward(at<const T>(y), dim(y, 0), dim(y, 1), at<const T>(down_bias),
                             at<const int32_t>(offsets), experts_in(offsets), &norm,
                             at<const T>(scale), at<const T>(bias), at<const T>(weights),
                             at<T>(out), s));
}
template <typename T>
ffi::Error norm_backward_as(hipStream_t s, In dy, In index, In y, In down_bias, In offsets,
                            In scale, In bias, In weights, int64_t index_div,
                            const bux_norm& norm, Out& dv, Out& d_weights, Out& d_scale,
                            Out& d_bias, Out& ws) {
  return status(norm_backward(
      at<const T>(dy), at<const int32_t>(index), static_cast<int32_t>(index_div), dim(dy, 0),
      at<const T>(y), dim(y, 0), dim(y, 1), at<const T>(down_bias), at<const int32_t>(offsets),
      experts_in(offsets), &norm, at<const T>(scale), at<const T>(bias), at<const T>(weights),
      at<T>(dv), at<T>(d_weights), at<float>(d_scale), at<float>(d_bias), at<void>(ws),
      ws->size_bytes(), s));
}
}  // namespace

// x is aliased to the result (in place): the caller passes input_output_aliases={0: 0}.
static ffi::Error ExpertBiasAdd(hipStream_t s, In x, In bias, In offsets, Out x_out) {
  return f32(x) ? expert_bias_add_as<float>(s, bias, offsets, x_out)
                : expert_bias_add_as<uint16_t>(s, bias, offsets, x_out);
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(BuxExpertBiasAdd, ExpertBiasAdd,
                              ffi::Ffi::Bind().Ctx<Stream>().Arg<In>().Arg<In>().Arg<In>()
                                  .Ret<In>());

// index and weights may be empty; m = the index's entries, or x's rows.
static ffi::Error ExpertSums(hipStream_t s, In x, In index, In weights, In offsets,
                             int64_t index_div, Out out) {
  return f32(x) ? expert_sums_as<float>(s, x, index, weights, offsets, index_div, out)
                : expert_sums_as<uint16_t>(s, x, index, weights, offsets, index_div, out);
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(BuxExpertSums, ExpertSums,
                              ffi::Ffi::Bind().Ctx<Stream>().Arg<In>().Arg<In>().Arg<In>()
                                  .Arg<In>().Attr<int64_t>("index_div").Ret<In>());

// inverse [t, k]; weights are the sorted rows'.
static ffi::Error TokenSumsBiased(hipStream_t s, In y, In inverse, In bias, In offsets,
                                  In weights, Out out) {
  return f32(y) ? token_sums_biased_as<float>(s, y, inverse, bias, offsets, weights, out)
                : token_sums_biased_as<uint16_t>(s, y, inverse, bias, offsets, weights, out);
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(BuxTokenSumsBiased, TokenSumsBiased,
                              ffi::Ffi::Bind().Ctx<Stream>().Arg<In>().Arg<In>().Arg<In>()
                                  .Arg<In>().Arg<In>().Ret<In>());

// d_weights is aliased to the result (added to in place): input_output_aliases={4: 0}.
static ffi::Error ExpertBiasWeightGrad(hipStream_t s, In dy, In index, In bias, In offsets,
                                       In d_weights, int64_t index_div, Out d_weights_out) {
  (void)d_weights;
  return f32(dy) ? bias_weight_grad_as<float>(s, dy, index, bias, offsets, index_div, d_weights_out)
                 : bias_weight_grad_as<uint16_t>(s, dy, index, bias, offsets, index_div,
                                                 d_weights_out);
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(BuxExpertBiasWeightGrad, ExpertBiasWeightGrad,
                              ffi::Ffi::Bind().Ctx<Stream>().Arg<In>().Arg<In>().Arg<In>()
                                  .Arg<In>().Arg<In>().Attr<int64_t>("index_div").Ret<In>());

// down_bias, scale and bias may be empty.
static ffi::Error ExpertNormForward(hipStream_t s, In y, In down_bias, In offsets, In scale,
                                    In bias, In weights, BUX_NORM_PARAMS, Out out) {
  const bux_norm norm = BUX_NORM;
  return f32(y) ? norm_forward_as<float>(s, y, down_bias, offsets, scale, bias, weights, norm, out)
                : norm_forward_as<uint16_t>(s, y, down_bias, offsets, scale, bias, weights, norm,
                                            out);
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(BuxExpertNormForward, ExpertNormForward,
                              ffi::Ffi::Bind().Ctx<Stream>().Arg<In>().Arg<In>().Arg<In>()
                                  .Arg<In>().Arg<In>().Arg<In>() BUX_NORM_ATTRS.Ret<In>());

static ffi::Error ExpertNormBackward(hipStream_t s, In dy, In index, In y, In down_bias,
                                     In offsets, In scale, In bias, In weights, int64_t index_div,
                                     BUX_NORM_PARAMS, Out dv, Out d_weights, Out d_scale,
                                     Out d_bias, Out ws) {
  const bux_norm norm = BUX_NORM;
  if (f32(y))
    return norm_backward_as<float>(s, dy, index, y, down_bias, offsets, scale, bias, weights,
                                   index_div, norm, dv, d_weights, d_scale, d_bias, ws);
  return norm_backward_as<uint16_t>(s, dy, index, y, down_bias, offsets, scale, bias, weights,
                                    index_div, norm, dv, d_weights, d_scale, d_bias, ws);
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(BuxExpertNormBackward, ExpertNormBackward,
                              ffi::Ffi::Bind().Ctx<Stream>().Arg<In>().Arg<In>().Arg<In>()
                                  .Arg<In>().Arg<In>().Arg<In>().Arg<In>().Arg<In>()
                                  .Attr<int64_t>("index_div") BUX_NORM_ATTRS.Ret<In>()
                                  .Ret<In>().Ret<In>().Ret<In>().Ret<In>());

// --- the router ----------------------------------------------------------------------
// x [t, d], kernel [d, n_logits]; bias and choice_bias may be empty, as may the sinks,
// scores and logits results.

static ffi::Error Route(hipStream_t s, In x, In kernel, In bias, In choice_bias,
                        float logit_scale, int64_t router, int64_t scored, int64_t groups,
                        int64_t keep, int64_t k, int64_t normalize, float scaling, Out idx,
                        Out weights, Out sinks, Out scores, Out logits, Out ws) {
  return status(bux_route(
      at<const uint16_t>(x), at<const uint16_t>(kernel), at<const float>(bias), dim(x, 0),
      dim(x, 1), static_cast<int32_t>(dim(kernel, 1)), logit_scale, static_cast<int>(router),
      static_cast<int32_t>(scored), at<const float>(choice_bias), static_cast<int32_t>(groups),
      static_cast<int32_t>(keep), static_cast<int32_t>(k), static_cast<int>(normalize), scaling,
      at<int32_t>(idx), at<uint16_t>(weights), at<uint16_t>(sinks), at<float>(scores),
      at<float>(logits), at<void>(ws), ws->size_bytes(), s));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(BuxRoute, Route,
                              ffi::Ffi::Bind().Ctx<Stream>().Arg<In>().Arg<In>().Arg<In>()
                                  .Arg<In>().Attr<float>("logit_scale").Attr<int64_t>("router")
                                  .Attr<int64_t>("scored").Attr<int64_t>("groups")
                                  .Attr<int64_t>("keep").Attr<int64_t>("k")
                                  .Attr<int64_t>("normalize").Attr<float>("scaling")
                                  .Ret<In>().Ret<In>().Ret<In>().Ret<In>().Ret<In>().Ret<In>());

// --- the MXFP8 wire rows ----------------------------------------------------------------

// packed [m, d + d/32]; index may be empty.
static ffi::Error MxPackRows(hipStream_t s, In x, In index, int64_t index_div, Out packed) {
  const int64_t d = dim(x, 1);
  return status(bux_mx_pack_rows(at<const uint16_t>(x), at<const int32_t>(index),
                                 static_cast<int32_t>(index_div), dim(x, 0), dim(packed, 0), d,
                                 at<uint8_t>(packed), s));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(BuxMxPackRows, MxPackRows,
                              ffi::Ffi::Bind().Ctx<Stream>().Arg<In>().Arg<In>()
                                  .Attr<int64_t>("index_div").Ret<In>());

static ffi::Error MxUnpackRows(hipStream_t s, In packed, Out out) {
  return status(bux_mx_unpack_rows(at<const uint8_t>(packed), dim(out, 0), dim(out, 1),
                                   at<uint16_t>(out), s));
}
XLA_FFI_DEFINE_HANDLER_SYMBOL(BuxMxUnpackRows, MxUnpackRows,
                              ffi::Ffi::Bind().Ctx<Stream>().Arg<In>().Ret<In>());

#endif  // __has_include("xla/ffi/api/ffi.h")
