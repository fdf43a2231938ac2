// ref_shim.cc -- extern "C" entry points over the reference's own CPU dequant
// (TEST INFRASTRUCTURE ONLY).
//
// Compiled by oracle/Makefile (target `ref`) together with the reference
// sources where they lie (/root/reference/src/quant.cc and common.cc, headers
// quant.h / dtypes.h / common.h), into oracle/_ref/libref_quant.so. Nothing from
// the reference is copied into this repository; this file only forwards.
// Used to validate the oracle's restatement (tests/test_oracle.py) and to write
// the golden vectors under tests/golden/.
#include <chrono>
#include <cstdint>

#include "dtypes.h"
#include "quant.h"

extern "C" {

// rpg::DequantizeRow, src/quant.cc:416-436. Returns 0, or -1 if it threw.
int ref_dequantize_row(uint32_t type, const uint8_t* src, int64_t n_elems, float* dst) {
  try {
    rpg::DequantizeRow(type, src, n_elems, dst);
    return 0;
  } catch (...) {
    return -1;
  }
}

// rpg::TypeRowBytes, src/quant.cc:406-414; -1 if it threw.
int64_t ref_type_row_bytes(uint32_t type, int64_t n_elems) {
  try {
    return rpg::TypeRowBytes(type, n_elems);
  } catch (...) {
    return -1;
  }
}

// rpg::F16ToF32, src/dtypes.h:21-47, over an array (results stay in memory, so
// NaN payloads are not disturbed by a float return through a foreign call).
void ref_f16_to_f32_array(const uint16_t* src, int64_t n, float* dst) {
  for (int64_t i = 0; i < n; ++i) dst[i] = rpg::F16ToF32(src[i]);
}

// rpg::F32ToF16, src/dtypes.h:50-76 (ties away from zero; kept to show it is
// not the KV write's rounding).
uint16_t ref_f32_to_f16_dtypes(float f) { return rpg::F32ToF16(f); }

// The CPU engine's embedding gather as the reference's CPU path runs it: one
// rpg::DequantizeRow per token row (src/quant.cc:416-436), one thread, timed
// here so no foreign-call overhead enters the figure. Returns the best of
// `reps` wall-clock seconds, or -1 if a row threw.
double ref_bench_gather(uint32_t type, const uint8_t* table, int64_t row_bytes, const int32_t* ids, int64_t seq,
                        int64_t cols, float* out, int reps) {
  double best = -1.0;
  for (int r = 0; r < reps; ++r) {
    const auto t0 = std::chrono::steady_clock::now();
    try {
      for (int64_t t = 0; t < seq; ++t) {
        rpg::DequantizeRow(type, table + static_cast<int64_t>(ids[t]) * row_bytes, cols, out + t * cols);
      }
    } catch (...) {
      return -1.0;
    }
    const double s = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    if (best < 0 || s < best) best = s;
  }
  return best;
}

}  // extern "C"
