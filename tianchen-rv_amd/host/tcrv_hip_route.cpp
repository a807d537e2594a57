// tcrv_hip_route.cpp -- the host-side HIP provider of TianChen-RV's
// contraction path: typed facts -> gfx950 algorithm, and op identity -> the
// libtcrv_hip entry point with its runtime-ABI parameters.  Host C++ only;
// every launch goes through the C-ABI of libtcrv_hip.
#include "tcrv_hip_route.h"

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <iterator>
#include <string>

namespace tianchenrv::plugin::hip {
namespace {

// Fact 1: libtcrv_hip has a gfx950 kernel for this weight block format.  The
// K-quants have none (out of this path's scope), so the request is declined
// and stays on the caller's existing route.
bool hipKernelExists(QuantType weight) {
  switch (weight) {
  case QuantType::Q4_0:
  case QuantType::Q8_0:
    return true;
  case QuantType::Q4_K:
    return false;
  }
  return false;
}

// Fact 2: the weights already sit in the x16 interleave.  Decode runs the
// repacked GEMV; prefill runs the repack GEMM, which the reference defines for
// Q4_0 only (tcrv_rvv.repack_gemm_q4_0_q8_0, RVVOps.td:4228), so a Q8_0 x16
// prefill is declined rather than silently unpacked.
bool weightsAreX16(WeightLayout layout) { return layout == WeightLayout::BlockX16; }

// Fact 3: decode is one activation row: the weight stream is read once and
// the work is HBM-bound, so it runs as a GEMV; prefill is a dense contraction
// and runs on the int8 matrix cores.
bool isDecode(MRegime m) { return m == MRegime::Decode; }

const char *gemmEntry(QuantType weight) {
  return weight == QuantType::Q4_0 ? "tcrv_hip_q4_0_q8_0_gemm" : "tcrv_hip_q8_0_q8_0_gemm";
}

const char *repackEntry(QuantType weight) {
  return weight == QuantType::Q4_0 ? "tcrv_hip_repack_gemv_q4_0_q8_0"
                                   : "tcrv_hip_repack_gemv_q8_0_q8_0";
}

}  // namespace

HipContractionSelection selectHipContractionAlgorithm(QuantType weight, MRegime mRegime,
                                                      WeightLayout layout) {
  if (!hipKernelExists(weight))
    return {HipContractionAlgorithm::Decline, "hip-decline-no-gfx950-kernel-for-quant", nullptr};
  if (weightsAreX16(layout)) {
    if (isDecode(mRegime))
      return {HipContractionAlgorithm::RepackGemv, weight == QuantType::Q4_0
                                                       ? "hip-repack-gemv-q4_0x16-decode"
                                                       : "hip-repack-gemv-q8_0x16-decode",
              repackEntry(weight)};
    if (weight == QuantType::Q4_0)
      return {HipContractionAlgorithm::RepackGemm, "hip-repack-gemm-q4_0x16-prefill-mfma-i8",
              "tcrv_hip_repack_gemm_q4_0_q8_0"};
    return {HipContractionAlgorithm::Decline, "hip-decline-q8_0x16-prefill-no-repack-gemm",
            nullptr};
  }
  if (isDecode(mRegime))
    return {HipContractionAlgorithm::DecodeGemv,
            weight == QuantType::Q4_0 ? "hip-decode-gemv-q4_0-hbm-bound"
                                      : "hip-decode-gemv-q8_0-hbm-bound",
            gemmEntry(weight)};
  return {HipContractionAlgorithm::MfmaGemm,
          weight == QuantType::Q4_0 ? "hip-prefill-mfma-i8-gemm-q4_0-decoded-at-staging"
                                    : "hip-prefill-mfma-i8-gemm-q8_0",
          gemmEntry(weight)};
}

MRegime deriveMRegime(size_t nc) { return nc <= 1 ? MRegime::Decode : MRegime::Prefill; }

HipBinarySelection selectHipBinary(int kind, int elem) {
  // kind: the verifier's set, "add" | "sub" | "mul"
  // (RVVDialectArithmeticOps.cpp:58-61), the intrinsic family chosen by
  // binaryMnemonic (RVVToEmitC.cpp:4976-4993); elem: every element type the
  // kernel is built for (signed and unsigned integers of 8-64 bits wrap alike,
  // f32/f64 are single IEEE operations)
  if (kind < TCRV_HIP_BINARY_ADD || kind > TCRV_HIP_BINARY_MUL)
    return {nullptr, "hip-decline-binary-kind-outside-add-sub-mul"};
  if (elem < TCRV_HIP_ELEM_I8 || elem > TCRV_HIP_ELEM_F64)
    return {nullptr, "hip-decline-binary-element-type"};
  const bool fp = elem == TCRV_HIP_ELEM_F32 || elem == TCRV_HIP_ELEM_F64;
  return {"tcrv_hip_binary", fp ? "hip-binary-float-ieee" : "hip-binary-integer-wrapping"};
}

namespace {

struct AbiParam {
  const char *cName;
  const char *cType;
  const char *role;
};

struct HipKernelRoute {
  const char *op;
  const char *entry;
  AbiParam params[9];
  size_t nparams;
};

// Parameter names, C types and roles as the reference's fixtures declare them
// (test/Conversion/RVV/...):
//   binary:         rvv-to-emitc-add-cpp-golden.mlir:15-18 (lhs, rhs, out, n)
//   integer core:   rvv-to-emitc-packed-i4-offset-binary-x-i8-product-reduce.mlir:22-27
//   q8_0 block dot: rvv-to-emitc-q8-0-q8-0-block-dot.mlir:16-19
//   q4_0 block dot: rvv-to-emitc-q4-0-q8-0-block-dot.mlir:24-31
//   q4_0 gemm:      rvv-to-emitc-q4-0-q8-0-gemm.mlir:23-31
//   q4_0 gemm tile: rvv-to-emitc-q4-0-q8-0-gemm-tile.mlir (+ its activation_cols)
//   repack gemvs:   rvv-to-emitc-repack-gemv-q4-0-q8-0.mlir:26-30,
//                   rvv-to-emitc-repack-gemv-q8-0-q8-0-vlen256.mlir
//   repack gemm:    rvv-to-emitc-repack-gemm-q4-0-q8-0.mlir:22-28
//   pack:           rvv-to-emitc-pack-q4-0-to-q4-0x16.mlir:19-21
//   quantize:       rvv-to-emitc-ggml-quantize-row-q8-0.mlir
// The Q8_0 GEMM has no reference op; it takes the q4_0 GEMM's ABI with Q8_0
// weights.  Nor do the block dequants (tcrv_rvv.dequantize, RVVOps.td:
// 8601-8632, is i32 -> f32 with one scale): their rows are keyed by the ggml
// function they restate (ggml.dequantize_row_q8_0 / _q4_0) and take its
// parameters (x, y, k) as (vx, y, n).  A row is found by its exact op identity (the op name); nothing is
// read from a name beyond that.
constexpr const char *kN = "runtime-element-count";
constexpr const char *kOut = "output-buffer";
constexpr const char *kLhs = "lhs-input-buffer";
constexpr const char *kRhs = "rhs-input-buffer";
// Not runtime-ABI values in the reference: an op attribute the emitted C bakes
// in (q4_0_q8_0_gemm_tile's activation_cols, tcrv_rvv.binary's kind) and the
// element type of the op's vectors, passed at run time here.
constexpr const char *kOpAttr = "op-attribute";
constexpr const char *kElemType = "element-type";

const HipKernelRoute kHipKernelRoutes[] = {
    // tcrv_rvv.binary: the op's kind attribute and element type are typed
    // facts (tcrv_hip_route_binary validates them); the entry takes them as its
    // first two arguments, then the reference's (lhs, rhs, out, n)
    {"tcrv_rvv.binary", "tcrv_hip_binary",
     {{"kind", "int", kOpAttr}, {"elem", "int", kElemType}, {"lhs", "const void *", kLhs},
      {"rhs", "const void *", kRhs}, {"out", "void *", kOut}, {"n", "size_t", kN}},
     6},
    {"tcrv_rvv.packed_i4_offset_binary_x_i8_product",
     "tcrv_hip_packed_i4_offset_binary_x_i8_product_reduce",
     {{"w", "const int8_t *", kLhs}, {"qlo", "const int8_t *", kRhs},
      {"qhi", "const int8_t *", kRhs}, {"acc", "const int32_t *", "accumulator-input-buffer"},
      {"out", "int32_t *", kOut}, {"n", "size_t", kN}},
     6},
    {"tcrv_rvv.q4_0_q8_0_block_dot", "tcrv_hip_q4_0_q8_0_block_dot",
     {{"n", "size_t", kN}, {"s", "float *", kOut}, {"bs", "size_t", "output-stride"},
      {"vx", "const uint8_t *", kLhs}, {"bx", "size_t", "lhs-input-stride"},
      {"vy", "const uint8_t *", kRhs}, {"by", "size_t", "rhs-input-stride"},
      {"nrc", "int32_t", "rhs-scalar-value"}},
     8},
    {"tcrv_rvv.q4_0_q8_0_gemm", "tcrv_hip_q4_0_q8_0_gemm",
     {{"n", "size_t", kN}, {"s", "float *", kOut}, {"vx", "const uint8_t *", kLhs},
      {"vy", "const uint8_t *", kRhs}, {"by", "size_t", "rhs-input-stride"},
      {"nr", "size_t", "source-byte-stride"}, {"nc", "size_t", "destination-byte-stride"},
      {"bx", "size_t", "lhs-input-stride"}, {"bs", "size_t", "output-stride"}},
     9},
    {"tcrv_rvv.q4_0_q8_0_gemm_tile", "tcrv_hip_q4_0_q8_0_gemm_tile",
     {{"n", "size_t", kN}, {"s", "float *", kOut}, {"vx", "const uint8_t *", kLhs},
      {"vy", "const uint8_t *", kRhs}, {"by", "size_t", "rhs-input-stride"},
      {"m", "size_t", kOpAttr}},
     6},
    {"tcrv_rvv.repack_gemv_q4_0_q8_0", "tcrv_hip_repack_gemv_q4_0_q8_0",
     {{"n", "size_t", kN}, {"s", "float *", kOut}, {"vx", "const uint8_t *", kLhs},
      {"vy", "const uint8_t *", kRhs}, {"nc", "size_t", "destination-byte-stride"}},
     5},
    {"tcrv_rvv.repack_gemm_q4_0_q8_0", "tcrv_hip_repack_gemm_q4_0_q8_0",
     {{"n", "size_t", kN}, {"s", "float *", kOut}, {"vx", "const uint8_t *", kLhs},
      {"vy", "const uint8_t *", kRhs}, {"nr", "size_t", "source-byte-stride"},
      {"nc", "size_t", "destination-byte-stride"}, {"bs", "size_t", "output-stride"}},
     7},
    {"tcrv_rvv.pack_q4_0_to_q4_0x16", "tcrv_hip_pack_q4_0_to_q4_0x16",
     {{"nblocks", "size_t", kN}, {"src", "const uint8_t *", kLhs}, {"dst", "uint8_t *", kOut}},
     3},
    {"tcrv_rvv.repack_gemv_q8_0_q8_0", "tcrv_hip_repack_gemv_q8_0_q8_0",
     {{"n", "size_t", kN}, {"s", "float *", kOut}, {"vx", "const uint8_t *", kLhs},
      {"vy", "const uint8_t *", kRhs}, {"nc", "size_t", "destination-byte-stride"}},
     5},
    {"tcrv_rvv.q8_0_q8_0_block_dot", "tcrv_hip_q8_0_q8_0_block_dot",
     {{"n", "size_t", kN}, {"s", "float *", kOut}, {"vx", "const uint8_t *", kLhs},
      {"vy", "const uint8_t *", kRhs}},
     4},
    {"tcrv_rvv.q8_0_q8_0_gemm", "tcrv_hip_q8_0_q8_0_gemm",
     {{"n", "size_t", kN}, {"s", "float *", kOut}, {"vx", "const uint8_t *", kLhs},
      {"vy", "const uint8_t *", kRhs}, {"by", "size_t", "rhs-input-stride"},
      {"nr", "size_t", "source-byte-stride"}, {"nc", "size_t", "destination-byte-stride"},
      {"bx", "size_t", "lhs-input-stride"}, {"bs", "size_t", "output-stride"}},
     9},
    {"tcrv_rvv.quantize_row_q8_0", "tcrv_hip_quantize_row_q8_0",
     {{"n", "size_t", kN}, {"x", "const float *", kLhs}, {"vy", "uint8_t *", kOut}},
     3},
    {"ggml.dequantize_row_q8_0", "tcrv_hip_dequantize_row_q8_0",
     {{"vx", "const uint8_t *", kLhs}, {"y", "float *", kOut}, {"n", "size_t", kN}},
     3},
    {"ggml.dequantize_row_q4_0", "tcrv_hip_dequantize_row_q4_0",
     {{"vx", "const uint8_t *", kLhs}, {"y", "float *", kOut}, {"n", "size_t", kN}},
     3},
};
constexpr size_t kNumRoutes = std::size(kHipKernelRoutes);

// The schedule registry (tcrv_hip_route_schedule): for each knob of a kernel
// the legal candidates, the default and why.  Rows with an entry can be chosen
// per call, and bench.py (--only schedules) times every such candidate at the
// op's reference shapes; the rest are template constants of the library build,
// chosen by a sweep of rebuilt libraries.  The registry itself carries no
// timings (measured_us is -1).
const tcrv_hip_schedule kSchedules[] = {
    // the decode GEMV (q4_0 GEMM, nc = 1): rows per wave of the register-direct
    // kernel, 4 waves per work-group.  The fold runs on 8 lanes per row for 4
    // or 8 rows per wave, on 16 for 2.  The plain entry's own choice depends on
    // the shape: 2 up to 2048 weight rows (4 would leave too few work-groups to
    // cover the chip), 4 above; for rows of exactly 2048 or 1024 quants (n =
    // 2048, 1024) a knob of 4 selects the lane-group kernels, whose waves own 4
    // or 8 rows (2 or 4 lane groups of 32 or 16 lanes) by n and nr.
    {"tcrv_rvv.q4_0_q8_0_gemm", TCRV_HIP_M_DECODE, "gemv_q4_0_q8_0_direct", "rows_per_wave", 2,
     0, "tcrv_hip_gemv_q4_0_q8_0_shaped", -1.0,
     "2048 waves for 4096 rows: two per SIMD share the read, and the per-row fold chain has 15 "
     "lane hops; the plain entry's choice up to 2048 weight rows"},
    {"tcrv_rvv.q4_0_q8_0_gemm", TCRV_HIP_M_DECODE, "gemv_q4_0_q8_0_direct", "rows_per_wave", 4,
     1, "tcrv_hip_gemv_q4_0_q8_0_shaped", -1.0,
     "the default from 2049 weight rows (the 4096-row reference shape): one wave per SIMD, "
     "every lane busy in the decode and 32 fold lanes; at n = 2048 and 1024 the lane-group "
     "kernels"},
    {"tcrv_rvv.q4_0_q8_0_gemm", TCRV_HIP_M_DECODE, "gemv_q4_0_q8_0_direct", "rows_per_wave", 8,
     0, "tcrv_hip_gemv_q4_0_q8_0_shaped", -1.0,
     "512 waves for 4096 rows leave half the SIMDs idle during the read"},
    // the tiled GEMMs: tokens per work-group tile; the entries pick per shape:
    // 64 x 64 tiles of one 32 x 32 tile a wave where 256 x 128 tiles would not
    // fill one round of the CUs (at most 1024 work-groups), else 256 weight
    // rows and the larger tile when its rounds of 256 work-groups x 15 are at
    // most the smaller tile's rounds x 8 (one round of 256 x 256 tiles takes
    // ~1.87 rounds of 256 x 128 ones)
    {"tcrv_rvv.q8_0_q8_0_gemm", TCRV_HIP_M_PREFILL, "gemm_tiles32", "work_group_tokens", 64, 0,
     nullptr, -1.0,
     "one 32x32 tile a wave, operands straight from the records; where few output tiles "
     "(4096 x 128 x 4096: 72 -> 17 us pre-packed); from plain rows gemm_rows_few"},
    {"tcrv_rvv.q4_0_q8_0_gemm", TCRV_HIP_M_PREFILL, "gemm_tiles32", "work_group_tokens", 64, 0,
     nullptr, -1.0, "one 32x32 tile a wave; where few output tiles (4096 x 128: 86 -> 20 us)"},
    {"tcrv_rvv.q8_0_q8_0_gemm", TCRV_HIP_M_PREFILL, "gemm_tiles_q8", "work_group_tokens", 128, 0,
     nullptr, -1.0,
     "16 waves of two 32x32 tiles, 6-block K chunks; where it takes fewer rounds (4096 x 2048 "
     "outputs: one round)"},
    {"tcrv_rvv.q8_0_q8_0_gemm", TCRV_HIP_M_PREFILL, "gemm_tiles256_q8", "work_group_tokens", 256,
     1, nullptr, -1.0,
     "8 waves of 2 x 4 32x32 tiles, 4-block K chunks: half the LDS operand reads and a third fewer "
     "DMA instructions per tile and block; the 4096^3 reference shape is one round"},
    {"tcrv_rvv.q4_0_q8_0_gemm", TCRV_HIP_M_PREFILL, "gemm_tiles_q4", "work_group_tokens", 128, 0,
     nullptr, -1.0, "16 waves of two transposed 32x32 tiles; where it takes fewer rounds"},
    {"tcrv_rvv.q4_0_q8_0_gemm", TCRV_HIP_M_PREFILL, "gemm_tiles256_q4", "work_group_tokens", 256,
     1, nullptr, -1.0,
     "8 waves of 2 x 4 transposed tiles, a token tile's d_y read once for both weight tiles"},
    // the 256 x 128 tiled Q8_0 GEMM: blocks per K chunk (two LDS stages for
    // 5-6 blocks, three for 3-4; the 256 x 256 kernel fits two stages of 4);
    // a build-time constant
    {"tcrv_rvv.q8_0_q8_0_gemm", TCRV_HIP_M_PREFILL, "gemm_tiles_q8", "k_chunk_blocks", 3, 0,
     nullptr, -1.0, "three stages; the most barriers per K"},
    {"tcrv_rvv.q8_0_q8_0_gemm", TCRV_HIP_M_PREFILL, "gemm_tiles_q8", "k_chunk_blocks", 4, 0,
     nullptr, -1.0, "three stages"},
    {"tcrv_rvv.q8_0_q8_0_gemm", TCRV_HIP_M_PREFILL, "gemm_tiles_q8", "k_chunk_blocks", 5, 0,
     nullptr, -1.0, "two stages; even with 6 in the sweep"},
    {"tcrv_rvv.q8_0_q8_0_gemm", TCRV_HIP_M_PREFILL, "gemm_tiles_q8", "k_chunk_blocks", 6, 1,
     nullptr, -1.0,
     "fastest in the sweep with 5 (two stages, 154 KB of LDS: one chunk in flight covers the DMA "
     "latency); 6 divides the 128 blocks of K = 4096 more evenly"},
    // quantize_row_q8_0: 32-float blocks per 8-lane group; a build-time constant
    {"tcrv_rvv.quantize_row_q8_0", -1, "quantize_q8_0", "blocks_per_lane_group", 1, 0, nullptr,
     -1.0, "fewer loads in flight per thread"},
    {"tcrv_rvv.quantize_row_q8_0", -1, "quantize_q8_0", "blocks_per_lane_group", 2, 1, nullptr,
     -1.0, "fastest in the sweep"},
    {"tcrv_rvv.quantize_row_q8_0", -1, "quantize_q8_0", "blocks_per_lane_group", 4, 0, nullptr,
     -1.0, "more registers, fewer waves"},
    // tcrv_rvv.binary (add f32, n = 2^24): 16-byte vectors per operand and
    // thread; a build-time constant
    {"tcrv_rvv.binary", -1, "add_f32_vec4", "vectors_per_thread", 1, 0, nullptr, -1.0,
     "loads of one vector in flight"},
    {"tcrv_rvv.binary", -1, "add_f32_vec4", "vectors_per_thread", 2, 1, nullptr, -1.0,
     "fastest in the sweep"},
    {"tcrv_rvv.binary", -1, "add_f32_vec4", "vectors_per_thread", 4, 0, nullptr, -1.0,
     "fewer work-groups in flight"},
    {"tcrv_rvv.binary", -1, "add_f32_vec4", "vectors_per_thread", 8, 0, nullptr, -1.0,
     "fewer work-groups in flight"},
};
constexpr size_t kNumSchedules = std::size(kSchedules);

// The C element type a tcrv_rvv.binary of element `elem` reads and writes.
const char *binaryCType(int elem) {
  switch (elem) {
  case TCRV_HIP_ELEM_I8: return "int8_t";
  case TCRV_HIP_ELEM_U8: return "uint8_t";
  case TCRV_HIP_ELEM_I16: return "int16_t";
  case TCRV_HIP_ELEM_U16: return "uint16_t";
  case TCRV_HIP_ELEM_I32: return "int32_t";
  case TCRV_HIP_ELEM_U32: return "uint32_t";
  case TCRV_HIP_ELEM_I64: return "int64_t";
  case TCRV_HIP_ELEM_F32: return "float";
  case TCRV_HIP_ELEM_F64: return "double";
  default: return nullptr;
  }
}

const char *binaryKindName(int kind) {
  switch (kind) {
  case TCRV_HIP_BINARY_ADD: return "TCRV_HIP_BINARY_ADD";
  case TCRV_HIP_BINARY_SUB: return "TCRV_HIP_BINARY_SUB";
  case TCRV_HIP_BINARY_MUL: return "TCRV_HIP_BINARY_MUL";
  default: return nullptr;
  }
}

const char *binaryElemName(int elem) {
  static const char *const names[] = {"TCRV_HIP_ELEM_I8",  "TCRV_HIP_ELEM_U8",  "TCRV_HIP_ELEM_I16",
                                      "TCRV_HIP_ELEM_U16", "TCRV_HIP_ELEM_I32", "TCRV_HIP_ELEM_U32",
                                      "TCRV_HIP_ELEM_I64", "TCRV_HIP_ELEM_F32", "TCRV_HIP_ELEM_F64"};
  return elem >= TCRV_HIP_ELEM_I8 && elem <= TCRV_HIP_ELEM_F64 ? names[elem] : nullptr;
}

// The exported function of one route row: its parameters are the row's
// runtime-ABI parameters (op attributes and the element type excluded: the
// emitted C bakes those in, so they come from `attrs`) plus the stream; its
// body forwards to the row's libtcrv_hip entry.  `declaration` emits the
// prototype alone.  Returns false for missing or invalid attributes.
bool exportFunction(const HipKernelRoute &r, const std::string &name, const int64_t *attrs,
                    size_t nattrs, bool declaration, std::string &out) {
  const bool binary = std::strcmp(r.op, "tcrv_rvv.binary") == 0;
  const bool tile = std::strcmp(r.op, "tcrv_rvv.q4_0_q8_0_gemm_tile") == 0;
  const size_t need = binary ? 2 : tile ? 1 : 0;
  if (nattrs < need || (need && !attrs))
    return false;
  const char *elemType = nullptr;
  if (binary) {
    elemType = binaryCType(static_cast<int>(attrs[1]));
    if (!binaryKindName(static_cast<int>(attrs[0])) || !elemType)
      return false;
  }
  if (tile && attrs[0] < 1)
    return false;
  std::string sig, call;
  for (size_t i = 0; i < r.nparams; ++i) {
    const AbiParam &p = r.params[i];
    if (!call.empty())
      call += ", ";
    if (std::strcmp(p.role, kOpAttr) == 0 || std::strcmp(p.role, kElemType) == 0) {
      if (binary)
        call += std::strcmp(p.cName, "kind") == 0 ? binaryKindName(static_cast<int>(attrs[0]))
                                                  : binaryElemName(static_cast<int>(attrs[1]));
      else
        call += std::to_string(attrs[0]) + " /* " + p.cName + " */";
      continue;
    }
    std::string ctype = p.cType;
    if (binary && ctype.find("void") != std::string::npos)  // the element's C type
      ctype = (ctype.rfind("const ", 0) == 0 ? std::string("const ") : std::string()) +
              elemType + " *";
    if (!sig.empty())
      sig += ", ";
    sig += ctype + (ctype.back() == '*' ? "" : " ") + p.cName;
    call += p.cName;
  }
  const std::string proto =
      "extern \"C\" int " + name + "(" + sig + (sig.empty() ? "" : ", ") + "void *stream)";
  if (declaration) {
    out += proto + ";\n";
    return true;
  }
  out += "// ";
  out += r.op;
  out += " -> libtcrv_hip ";
  out += r.entry;
  out += "\n" + proto + " {\n  return " + r.entry + "(" + call + ", stream);\n}\n";
  return true;
}

bool validFacts(int quant, int regime, int layout) {
  return quant >= TCRV_HIP_QUANT_Q4_0 && quant <= TCRV_HIP_QUANT_Q4_K &&
         (regime == TCRV_HIP_M_DECODE || regime == TCRV_HIP_M_PREFILL) &&
         (layout == TCRV_HIP_LAYOUT_PLAIN || layout == TCRV_HIP_LAYOUT_X16);
}

}  // namespace
}  // namespace tianchenrv::plugin::hip

using namespace tianchenrv::plugin::hip;

extern "C" {

int tcrv_hip_route_select(int weight_quant, int m_regime, int weight_layout, int *algorithm,
                          const char **reason, const char **entry) {
  if (!validFacts(weight_quant, m_regime, weight_layout))
    return TCRV_HIP_ERR_BAD_SIZE;
  const HipContractionSelection sel = selectHipContractionAlgorithm(
      static_cast<QuantType>(weight_quant), static_cast<MRegime>(m_regime),
      static_cast<WeightLayout>(weight_layout));
  if (algorithm)
    *algorithm = static_cast<int>(sel.algorithm);
  if (reason)
    *reason = sel.reason;
  if (entry)
    *entry = sel.entry;
  return TCRV_HIP_OK;
}

int tcrv_hip_route_m_regime(size_t nc) { return static_cast<int>(deriveMRegime(nc)); }

int tcrv_hip_route_binary(int kind, int elem, const char **entry, const char **reason) {
  const HipBinarySelection sel = selectHipBinary(kind, elem);
  if (entry)
    *entry = sel.entry;
  if (reason)
    *reason = sel.reason;
  return sel.entry ? TCRV_HIP_OK : TCRV_HIP_ERR_UNSUPPORTED;
}

int tcrv_hip_route_contraction(int weight_quant, int weight_layout, size_t n, float *s,
                               const uint8_t *vx, const uint8_t *vy, size_t by, size_t nr,
                               size_t nc, size_t bx, size_t bs, void *stream, int *algorithm) {
  const int regime = static_cast<int>(deriveMRegime(nc));
  if (!validFacts(weight_quant, regime, weight_layout))
    return TCRV_HIP_ERR_BAD_SIZE;
  const HipContractionSelection sel = selectHipContractionAlgorithm(
      static_cast<QuantType>(weight_quant), static_cast<MRegime>(regime),
      static_cast<WeightLayout>(weight_layout));
  if (algorithm)
    *algorithm = static_cast<int>(sel.algorithm);
  const bool q4 = weight_quant == TCRV_HIP_QUANT_Q4_0;
  switch (sel.algorithm) {
  case HipContractionAlgorithm::Decline:
    return TCRV_HIP_ERR_UNSUPPORTED;
  case HipContractionAlgorithm::RepackGemv:
    if (nr == 0 || nc == 0)
      return TCRV_HIP_OK;
    if (nr % 16 != 0 || (nr > 1 && bs != 1))
      return TCRV_HIP_ERR_UNSUPPORTED;
    return q4 ? tcrv_hip_repack_gemv_q4_0_q8_0(n, s, vx, vy, nr, stream)
              : tcrv_hip_repack_gemv_q8_0_q8_0(n, s, vx, vy, nr, stream);
  case HipContractionAlgorithm::RepackGemm:
    // the selected kernel has a different contract from this call's GEMM ABI
    // (block_q8_0x4 activations, activation-row-major output s[col*bs + ir]):
    // refused here, the caller runs sel.entry in its own ABI
    return TCRV_HIP_ERR_UNSUPPORTED;
  case HipContractionAlgorithm::DecodeGemv:
  case HipContractionAlgorithm::MfmaGemm:
    return q4 ? tcrv_hip_q4_0_q8_0_gemm(n, s, vx, vy, by, nr, nc, bx, bs, stream)
              : tcrv_hip_q8_0_q8_0_gemm(n, s, vx, vy, by, nr, nc, bx, bs, stream);
  }
  return TCRV_HIP_ERR_UNSUPPORTED;
}

size_t tcrv_hip_route_count(void) { return kNumRoutes; }

const char *tcrv_hip_route_op(size_t row) {
  return row < kNumRoutes ? kHipKernelRoutes[row].op : nullptr;
}

const char *tcrv_hip_route_entry(size_t row) {
  return row < kNumRoutes ? kHipKernelRoutes[row].entry : nullptr;
}

size_t tcrv_hip_route_param_count(size_t row) {
  return row < kNumRoutes ? kHipKernelRoutes[row].nparams : 0;
}

int tcrv_hip_route_param(size_t row, size_t param, const char **c_name, const char **c_type,
                         const char **role) {
  if (row >= kNumRoutes || param >= kHipKernelRoutes[row].nparams)
    return TCRV_HIP_ERR_BAD_SIZE;
  const AbiParam &p = kHipKernelRoutes[row].params[param];
  if (c_name)
    *c_name = p.cName;
  if (c_type)
    *c_type = p.cType;
  if (role)
    *role = p.role;
  return TCRV_HIP_OK;
}

const char *tcrv_hip_export_prologue(void) {
  return "// Generated by the TianChen-RV HIP target export (libtcrv_hip_route): one\n"
         "// tcrv_emitc_<kernel>_<variant> per selected variant, forwarding to libtcrv_hip.\n"
         "#include <stddef.h>\n#include <stdint.h>\n\n#include \"tcrv_hip.h\"\n";
}

int tcrv_hip_export_function(const char *op, const char *kernel, const char *variant,
                             const int64_t *attrs, size_t nattrs, int form, char *buf, size_t cap,
                             size_t *needed) {
  if (!op || !kernel || !variant)
    return TCRV_HIP_ERR_NULL_POINTER;
  if (form != TCRV_HIP_EXPORT_DEFINITION && form != TCRV_HIP_EXPORT_DECLARATION)
    return TCRV_HIP_ERR_BAD_SIZE;
  const long row = tcrv_hip_route_find(op);
  if (row < 0)
    return TCRV_HIP_ERR_UNSUPPORTED;
  // the name the reference derives: tcrv_emitc_<kernel>_<variant>
  // (RVVToEmitC.cpp:167-172)
  const std::string name = std::string("tcrv_emitc_") + kernel + "_" + variant;
  std::string text;
  if (!exportFunction(kHipKernelRoutes[row], name, attrs, nattrs,
                      form == TCRV_HIP_EXPORT_DECLARATION, text))
    return TCRV_HIP_ERR_BAD_SIZE;
  if (needed)
    *needed = text.size() + 1;
  if (buf && cap > 0) {
    const size_t n = std::min(cap - 1, text.size());
    std::memcpy(buf, text.data(), n);
    buf[n] = '\0';
  }
  return TCRV_HIP_OK;
}

size_t tcrv_hip_route_schedule_count(void) { return kNumSchedules; }

int tcrv_hip_route_schedule(size_t index, tcrv_hip_schedule *out) {
  if (index >= kNumSchedules || !out)
    return TCRV_HIP_ERR_BAD_SIZE;
  *out = kSchedules[index];
  return TCRV_HIP_OK;
}

int tcrv_hip_route_schedule_default(const char *op, int m_regime, const char *knob,
                                    int64_t *value) {
  if (!op || !knob)
    return TCRV_HIP_ERR_UNSUPPORTED;
  for (const tcrv_hip_schedule &r : kSchedules)
    if (r.is_default && std::strcmp(r.op, op) == 0 && std::strcmp(r.knob, knob) == 0 &&
        (r.m_regime == -1 || r.m_regime == m_regime)) {
      if (value)
        *value = r.value;
      return TCRV_HIP_OK;
    }
  return TCRV_HIP_ERR_UNSUPPORTED;
}

long tcrv_hip_route_find(const char *op) {
  if (!op)
    return -1;
  for (size_t i = 0; i < kNumRoutes; ++i)
    if (std::strcmp(kHipKernelRoutes[i].op, op) == 0)
      return static_cast<long>(i);
  return -1;
}

}  // extern "C"
