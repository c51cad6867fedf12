// p0k_internal.h — host-side declarations shared by the runtime and the argument checker.
#pragma once
#include <string>

#include "../../include/p0k.h"

namespace p0k {
struct Params;
enum { K_MFMA = 0, K_GEMV = 1, K_GEMV_MF = 2, K_MFMA_DMA = 3 };
// kernel choice of one call: GEMV items are (128-column tile) x (K slice of KS), S slices per tile
struct Plan { int kernel, we, xm; unsigned bm, bn, S, KS; };
// validate a gemm call and translate it to kernel parameters (device pointers are filled in by the caller)
int prepare_gemm(const p0k_gemm_args *a, Params *out, Plan *plan, std::string *err);
int prepare_rowstats(const p0k_rowstats_args *a, std::string *err);
int prepare_pixstats(const p0k_pixstats_args *a, std::string *err);
struct AttnParams;
int prepare_attention(const p0k_attn_args *a, AttnParams *out, std::string *err);
// what: 1 = partial rows, 2 = finalize, 3 = both
int prepare_gn(const p0k_gn_args *a, int what, std::string *err);
}  // namespace p0k
