// Host-side internals shared by the bmx translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bmx.h"

namespace bmx {

// Records a message for bmx_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Converts the last HIP launch status into a bmx return code (0 or a
// positive hipError_t) and records its message.
int check_launch(const char* what);
int check_hip(hipError_t e, const char* what);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }
inline bool aligned(const void* p, uintptr_t a) {
  return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

// ---- qmv (M <= 8) -------------------------------------------------------
enum QmvEpilogue { QMV_STORE = 0, QMV_RESIDUAL = 1, QMV_SWIGLU = 2 };

struct QmvSegment {
  const uint32_t* w;  // [rows, K/8]
  const uint16_t* s;  // [rows, K/64]
  const uint16_t* b;  // [rows, K/64]
  uint16_t* y;        // [M, rows] (row stride = rows)
  int rows;
  int row0;  // first global output row of this segment
};

struct QmvParams {
  const uint16_t* x;  // [M, K], row stride ldx
  int64_t ldx;
  QmvSegment seg[3];
  int nseg;
  int m;  // rows of x (1..8)
  int N;  // total output rows over all segments (SWIGLU: rows of one matrix)
  int K;
  const uint16_t* res;     // QMV_RESIDUAL: [M, N] added to the product (may alias y)
  const uint16_t* norm_w;  // optional fused RMSNorm of x: weight [K]
  float eps;
  int kp;      // K columns staged in LDS per phase (set by launch_qmv)
  int sb_vec;  // s/b staged with 16-byte loads (set by launch_qmv)
};

// Validates shapes/alignment and launches the qmv kernel family.
int launch_qmv(QmvParams p, QmvEpilogue epi, hipStream_t stream);

}  // namespace bmx
