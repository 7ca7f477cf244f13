// Dense BF16 GEMM on the MFMA cores (uqm_dense.hip): the shared expert of
// calls with many tokens.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace uqm {

// out = x W^T for one dense BF16 matrix W (one weight matrix for every token).
//   kModeSilu: W = (gate, up), out bf16 [T, ldo] = bf16(silu(bf16(x Wg^T)) * bf16(x Wu^T))
//   kModeF32:  W = w[0],       out fp32 [split][T, ldo], K split over ksplit partials
// Rows W[r] start at w[m] + r * K (bf16 elements); x row t at x + t * ldx.
struct DenseArgs {
  const uint16_t* w[2];
  const uint16_t* x;
  int64_t ldx;
  int64_t rows;  // output rows (per matrix)
  int64_t K;     // input features (multiple of 64)
  int64_t T;     // tokens
  void* out;
  int64_t ldo;
  int64_t part_stride;  // elements between K-split partial outputs (kModeF32)
  int32_t ksplit;       // K-split partials (kModeF32 only; must divide K / 64)
};

// Smallest token count the dense kernel takes (a work item covers 128 or 256
// tokens).
constexpr int64_t kDenseMinTokens = 128;

bool dense_supported(int64_t rows, int64_t K, int64_t T);

// Workgroup size (4 or 8 waves: 128- or 256-token items) and K split (kModeF32
// only, at most max_split) with the least estimated time on cus CUs.
struct DensePlan {
  int waves;
  int ksplit;
};
DensePlan plan_dense(int nmat, int64_t rows, int64_t K, int64_t T, int cus, int max_split);

// nmat 2 = gate/up with the SiLU epilogue, 1 = FP32 rows; cus = compute units
// the persistent grid may take.
hipError_t launch_dense_mfma(int nmat, const DenseArgs& a, int waves, int cus, hipStream_t stream);

}  // namespace uqm
