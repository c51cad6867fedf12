// p0k_internal.h — host-side declarations shared by the runtime and the argument checker.
#pragma once
#include <string>

#include "../../include/p0k.h"

namespace p0k {
struct Params;
enum { K_MFMA = 0, K_GEMV = 1, K_GEMV_MF = 2, K_MFMA_DMA = 3, K_GEMV_SN = 4 };
// kernel choice of one call: GEMV items are (128-column tile) x (K slice of KS), S slices per tile
struct Plan { int kernel, we, xm; unsigned bm, bn, S, KS; bool mx, narrow; };
// What the kernel choice depends on besides the call: the device's CU count and the P0K_* tuning switches of the
// environment. A context reads them once (at creation and on p0k_ctx_reload_env); calls without a context read
// them on the spot.
struct Tuning {
  unsigned cus = 256;
  int gemv_mf = -1;            // P0K_GEMV_MF=0: the VALU stream for M > 1 (-1: not set)
  bool gemv_mq4 = true;        // P0K_GEMV_MQ4=0: q4 matrix-core decode with X' staged in LDS (k_gemv_mf)
  unsigned gemv_slices = 0;    // P0K_GEMV_SLICES=n: decode K slices (0: not set)
  unsigned gemv_mx = 4;        // P0K_GEMV_MX=n: q4 decode with 2..n rows on the stream kernel's matrix-core form
  bool gemv_narrow = true;     // P0K_GEMV_NARROW=0: no 64-column decode items (a K split fills the GPU instead)
  int gemv_sn = -1;            // P0K_GEMV_SN=0|1: short-call decode items of 16 rows never / wherever they apply
  bool mfma_reg = false;       // P0K_MFMA_KERNEL=reg: the register-staged MFMA kernel
  unsigned tile_m = 0, tile_n = 0;   // P0K_MFMA_TILE=MxN
  bool dma_tail = true;        // P0K_DMA_TAIL=0: one launch for a mostly empty last round
  int attn_bq = 0;             // P0K_ATTN_BQ=128|256
};
Tuning tuning_from_env(unsigned cus);
// validate a gemm call and translate it to kernel parameters (device pointers are filled in by the caller)
int prepare_gemm(const p0k_gemm_args *a, Params *out, Plan *plan, std::string *err, const Tuning &t);
int prepare_rowstats(const p0k_rowstats_args *a, std::string *err);
int prepare_pixstats(const p0k_pixstats_args *a, std::string *err);
struct AttnParams;
int prepare_attention(const p0k_attn_args *a, AttnParams *out, std::string *err);
// what: 1 = partial rows, 2 = finalize, 3 = both
int prepare_gn(const p0k_gn_args *a, int what, std::string *err);
}  // namespace p0k
