/*
 * tcrv_hip_route.h -- host-side HIP provider for TianChen-RV's contraction
 * path: which gfx950 kernel of libtcrv_hip runs a typed contraction request,
 * and the op-identity -> entry-point table a HIP emission driver would consult.
 *
 * The selection mirrors the reference's path-selection authority
 * `selectContractionAlgorithm(QuantType, MRegime, minVLEN)`
 * (include/TianChenRV/Plugin/RVV/RVVContractionPathSelection.h:24-66,
 * lib/Plugin/RVV/RVVContractionPathSelection.cpp:63-92): a pure function of
 * typed facts (the weight block format, the M regime of the op, and the weight
 * layout the stage-C materialization chose) returning an algorithm plus a
 * stable audit token.  It never matches on op-name strings.
 *
 * The route table mirrors the first-match kernel table of the RVV emitter
 * (kBlockDotKernels[], lib/Conversion/RVV/RVVToEmitC.cpp:338-423): one row per
 * op identity, carrying the libtcrv_hip entry point and the op's runtime-ABI
 * parameters in tcrv_rvv.runtime_abi_value declaration order (c_name, c_type,
 * role as the reference fixtures spell them), to which the HIP entry appends
 * one `void *stream`.
 *
 * libtcrv_hip_route.so is plain host C++ (no HIP headers) linked against
 * libtcrv_hip.so; the C functions below are its stable ABI.
 */
#ifndef TCRV_HIP_ROUTE_H
#define TCRV_HIP_ROUTE_H

#include <stddef.h>
#include <stdint.h>

#include "tcrv_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Typed facts (values of the C enums below are part of the ABI). */
enum { TCRV_HIP_QUANT_Q4_0 = 0, TCRV_HIP_QUANT_Q8_0 = 1, TCRV_HIP_QUANT_Q4_K = 2 };
enum { TCRV_HIP_M_DECODE = 0, TCRV_HIP_M_PREFILL = 1 };
enum { TCRV_HIP_LAYOUT_PLAIN = 0, TCRV_HIP_LAYOUT_X16 = 1 };
enum {
  TCRV_HIP_ALGO_DECLINE = 0,     /* no gfx950 kernel: the caller keeps its own route */
  TCRV_HIP_ALGO_DECODE_GEMV = 1, /* bandwidth-bound GEMV over plain rows */
  TCRV_HIP_ALGO_REPACK_GEMV = 2, /* GEMV over block_q*_0x16 weights */
  TCRV_HIP_ALGO_MFMA_GEMM = 3,   /* int8 MFMA GEMM */
  TCRV_HIP_ALGO_REPACK_GEMM = 4  /* int8 MFMA GEMM over block_q4_0x16 x block_q8_0x4 */
};

/* Selection from typed facts.  Writes the algorithm, its audit token and the
 * libtcrv_hip entry that runs it (NULL when declined); the strings have static
 * storage.  Returns TCRV_HIP_OK, or TCRV_HIP_ERR_BAD_SIZE for a value outside
 * the enums above (outputs untouched). */
TCRV_HIP_API int tcrv_hip_route_select(int weight_quant, int m_regime, int weight_layout,
                                       int *algorithm, const char **reason,
                                       const char **entry);

/* The M regime a shape implies when the op carries none: nc <= 1 is decode. */
TCRV_HIP_API int tcrv_hip_route_m_regime(size_t nc);

/* tcrv_rvv.binary from its typed facts: the op's `kind` attribute
 * (TCRV_HIP_BINARY_*) and its element type (TCRV_HIP_ELEM_*), the two facts
 * binaryMnemonic (RVVToEmitC.cpp:4976-4993) selects the RVV intrinsic from.
 * Writes the libtcrv_hip entry ("tcrv_hip_binary", taking (kind, elem, lhs,
 * rhs, out, n, stream)) and an audit token; returns TCRV_HIP_ERR_UNSUPPORTED
 * (entry NULL) for a kind or element type outside the grid. */
TCRV_HIP_API int tcrv_hip_route_binary(int kind, int elem, const char **entry,
                                       const char **reason);

/* Runs one contraction in the reference GEMM ABI
 * (n, s, vx, vy, by, nr, nc, bx, bs) -- q4_0_q8_0_gemm's parameter order,
 * test/Conversion/RVV/rvv-to-emitc-q4-0-q8-0-gemm.mlir:23-31 -- with that ABI's
 * meaning (activation column col at vy + col*by as plain Q8_0 rows, output
 * s[ir*bs + col]) on the algorithm tcrv_hip_route_select picks for
 * (weight_quant, the regime of nc, weight_layout).  x16 weights (vx holds nr/16
 * groups of 16 rows in the x16 layout, bx ignored, nr % 16 == 0) are served in
 * decode only: the repacked GEMV on one plain Q8_0 activation row, needing
 * bs == 1 (or nr == 1), writes s[ir].  An x16 prefill selects the repack GEMM
 * (tcrv_hip_repack_gemm_q4_0_q8_0), whose contract is not this ABI's
 * (block_q8_0x4 activations, output s[col*bs + ir]): this call refuses it, and
 * the caller runs that entry in its own ABI.  A declined or refused request, or
 * an x16 decode shape outside the above, returns TCRV_HIP_ERR_UNSUPPORTED before
 * touching anything.  *algorithm (may be NULL) receives the algorithm
 * selected. */
TCRV_HIP_API int tcrv_hip_route_contraction(int weight_quant, int weight_layout, size_t n,
                                            float *s, const uint8_t *vx, const uint8_t *vy,
                                            size_t by, size_t nr, size_t nc, size_t bx,
                                            size_t bs, void *stream, int *algorithm);

/* The op-identity route table.  Rows are numbered 0 .. count-1. */
TCRV_HIP_API size_t tcrv_hip_route_count(void);
/* Op identity (e.g. "tcrv_rvv.q8_0_q8_0_block_dot") and entry symbol of a row;
 * NULL for an index out of range. */
TCRV_HIP_API const char *tcrv_hip_route_op(size_t row);
TCRV_HIP_API const char *tcrv_hip_route_entry(size_t row);
/* Number of runtime-ABI parameters of a row (the entry takes one more: the
 * stream), or 0 for an index out of range. */
TCRV_HIP_API size_t tcrv_hip_route_param_count(size_t row);
/* Parameter `param` of a row: c_name, c_type and role strings as in the
 * reference fixtures.  Returns TCRV_HIP_OK or TCRV_HIP_ERR_BAD_SIZE. */
TCRV_HIP_API int tcrv_hip_route_param(size_t row, size_t param, const char **c_name,
                                      const char **c_type, const char **role);
/* Row of an op identity, or -1 when the table has none. */
TCRV_HIP_API long tcrv_hip_route_find(const char *op);

/* ---- schedule descriptors ------------------------------------------------
 * The reference looks a kernel's bounded schedule knobs up in a registry of
 * descriptors (lookupRVVScheduleDescriptor,
 * lib/Plugin/RVV/RVVScheduleDescriptorRegistry.cpp:151-190): the legal
 * candidate shapes, each with its knobs, and the default with the reason it
 * was chosen (measured-fastest, or a static cost); the knobs change how a
 * kernel runs, never what it computes (RVVOps.td:3912-3972).  This is the same
 * registry for the gfx950 kernels: one row per (op, regime, knob, candidate
 * value).  A row with a non-NULL `entry` names the libtcrv_hip entry that takes
 * the knob as an argument (every value bit-identical); the others are
 * build-time shapes.  The registry carries no timings: bench.py --only
 * schedules times every selectable candidate at the op's reference shapes, and
 * the tests check the defaults against a recorded run of it. */
typedef struct {
  const char *op;      /* op identity of the route table */
  int m_regime;        /* TCRV_HIP_M_DECODE or TCRV_HIP_M_PREFILL; -1: not regime-specific */
  const char *kernel;  /* the device kernel */
  const char *knob;    /* knob name */
  int64_t value;       /* the candidate's value */
  int is_default;      /* 1: the value the op's own entry runs */
  const char *entry;   /* entry taking the knob, or NULL (fixed at build time) */
  double measured_us;  /* -1: timings are measured by bench.py, not stored here */
  const char *reason;  /* why the default is the default, or how the candidate compares */
} tcrv_hip_schedule;
/* Number of rows, and row `index` (TCRV_HIP_ERR_BAD_SIZE past the end). */
TCRV_HIP_API size_t tcrv_hip_route_schedule_count(void);
TCRV_HIP_API int tcrv_hip_route_schedule(size_t index, tcrv_hip_schedule *out);
/* The default value of `knob` for (op, m_regime) (a row with m_regime -1
 * matches either regime); TCRV_HIP_ERR_UNSUPPORTED when the registry has none. */
TCRV_HIP_API int tcrv_hip_route_schedule_default(const char *op, int m_regime, const char *knob,
                                                 int64_t *value);

/* ---- the host half of the export (lib/Target for this backend) ----------
 * What a HIP emission driver hands to the artifact export in place of the RVV
 * C the reference renders with exportMaterializedEmitCModuleToCpp
 * (lib/Target/TargetArtifactExport.cpp:2040-2052): for one selected variant of
 * op `op`, the C++ text of
 *   extern "C" int tcrv_emitc_<kernel>_<variant>(<the op's runtime-ABI
 *                                                 parameters>, void *stream)
 * -- the name as the reference derives it (RVVToEmitC.cpp:167-172), the
 * parameters with the fixtures' names and C types in runtime_abi_value
 * declaration order (:134-145, :258-268) -- whose body forwards to the op's
 * libtcrv_hip entry and returns its status.  Op attributes the emitted C bakes
 * in are typed facts in attrs[]: tcrv_rvv.binary takes {kind, element}
 * (TCRV_HIP_BINARY_*, TCRV_HIP_ELEM_*), tcrv_rvv.q4_0_q8_0_gemm_tile
 * {activation_cols}.  form selects the definition or the prototype alone
 * (for a header).  Writes at most cap bytes, NUL-terminated, and the full size
 * in *needed (may be NULL).  Returns TCRV_HIP_ERR_UNSUPPORTED for an op outside
 * the table, TCRV_HIP_ERR_BAD_SIZE for missing or invalid attributes or form. */
enum { TCRV_HIP_EXPORT_DEFINITION = 0, TCRV_HIP_EXPORT_DECLARATION = 1 };
TCRV_HIP_API int tcrv_hip_export_function(const char *op, const char *kernel, const char *variant,
                                          const int64_t *attrs, size_t nattrs, int form,
                                          char *buf, size_t cap, size_t *needed);
/* The translation unit's opening text (includes), static storage. */
TCRV_HIP_API const char *tcrv_hip_export_prologue(void);

#ifdef __cplusplus
}  /* extern "C" */

namespace tianchenrv::plugin::hip {

/* The reference's path-selection enums (RVVContractionPathSelection.h:36-44). */
enum class QuantType { Q4_0 = TCRV_HIP_QUANT_Q4_0, Q8_0 = TCRV_HIP_QUANT_Q8_0, Q4_K = TCRV_HIP_QUANT_Q4_K };
enum class MRegime { Decode = TCRV_HIP_M_DECODE, Prefill = TCRV_HIP_M_PREFILL };
/* Plain ggml rows, or the block_q*_0x16 interleave the stage-C weight
 * materialization produces (pack_q4_0_to_q4_0x16, RVVOps.td:4551-4626). */
enum class WeightLayout { PlainRows = TCRV_HIP_LAYOUT_PLAIN, BlockX16 = TCRV_HIP_LAYOUT_X16 };

enum class HipContractionAlgorithm {
  Decline = TCRV_HIP_ALGO_DECLINE,
  DecodeGemv = TCRV_HIP_ALGO_DECODE_GEMV,
  RepackGemv = TCRV_HIP_ALGO_REPACK_GEMV,
  MfmaGemm = TCRV_HIP_ALGO_MFMA_GEMM,
  RepackGemm = TCRV_HIP_ALGO_REPACK_GEMM,
};

struct HipContractionSelection {
  HipContractionAlgorithm algorithm;
  const char *reason;  /* stable audit token */
  const char *entry;   /* libtcrv_hip symbol, nullptr when declined */
};

HipContractionSelection selectHipContractionAlgorithm(QuantType weight, MRegime mRegime,
                                                      WeightLayout layout);

struct HipBinarySelection {
  const char *entry;   /* libtcrv_hip symbol, nullptr when declined */
  const char *reason;  /* stable audit token */
};

HipBinarySelection selectHipBinary(int kind, int elem);

MRegime deriveMRegime(size_t nc);

}  // namespace tianchenrv::plugin::hip
#endif

#endif /* TCRV_HIP_ROUTE_H */
