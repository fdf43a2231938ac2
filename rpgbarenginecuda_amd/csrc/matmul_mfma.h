// Internal interface of the matrix-core prefill GEMM (k_matmul_mfma.hip), used
// by the GpuMatMulQuant entry points (k_matmul.hip).
#ifndef RPG_AMD_MATMUL_MFMA_H_
#define RPG_AMD_MATMUL_MFMA_H_

#include <cstdint>

namespace rpg {

// Activations scaled per token by a power of two and split into two fp16
// planes, plus the 32-column run sums (also split), in the library's split
// buffer (valid until the next split on the engine stream).
struct SplitActivations {
  void* planes = nullptr;       // 2 x [n_tokens][cols] fp16
  void* sums = nullptr;         // 2 x [n_tokens][cols / 32] fp16, planes sum_stride apart
  float* inv_scale = nullptr;   // [n_tokens]: 1 / s_t
  int64_t sum_stride = 0;       // fp16 elements between the two sum planes
  int64_t n_tokens = 0;
  int64_t cols = 0;
  // The split is launched by the first GEMM launch that reads it (beside that
  // matrix's weight decode when it takes the decoded-planes path); until then
  // x must stay unchanged.
  const float* x = nullptr;
  mutable bool pending = false;
};

// Prepares the split of x [n_tokens][cols] fp32 (16-byte aligned, cols % 32 ==
// 0) into the split buffer; the first LaunchMatMulMfmaSplit on it launches it.
SplitActivations SplitForMfma(const float* x, int64_t n_tokens, int64_t cols);

// OUT = X . W^T for one Q4_K / Q6_K matrix from split activations (cols =
// 256 nb; Q4_K rows 16-byte aligned, Q6_K 2-byte aligned).
void LaunchMatMulMfmaSplit(uint32_t type, const uint8_t* w, int64_t rows, int64_t row_bytes, int32_t nb,
                           const SplitActivations& sa, float* out);

// Split, then LaunchMatMulMfmaSplit.
void LaunchMatMulMfma(uint32_t type, const uint8_t* w, int64_t rows, int64_t row_bytes, int32_t nb, const float* x,
                      int64_t cols, int64_t n_tokens, float* out);

}  // namespace rpg

#endif  // RPG_AMD_MATMUL_MFMA_H_
