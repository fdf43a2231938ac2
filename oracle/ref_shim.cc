// ref_shim.cc -- extern "C" entry points over the reference's own CPU dequant
// (TEST INFRASTRUCTURE ONLY).
//
// Compiled by oracle/Makefile (target `ref`) together with the reference
// sources where they lie (/root/reference/src/quant.cc and common.cc, headers
// quant.h / dtypes.h / common.h), into oracle/_ref/libref_quant.so. Nothing from
// the reference is copied into this repository; this file only forwards.
// Used to validate the oracle's restatement (tests/test_oracle.py) and to write
// the golden vectors under tests/golden/.
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

}  // extern "C"
