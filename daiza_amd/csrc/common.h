// common.h — shared definitions of the gfx950 decode library (device + host).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "daiza_hip.h"

namespace dz {

// Q1_0 geometry (Daiza-engine/src/tensor/dtype.rs:11,14)
constexpr int kGroup = 128;      // weights per scale
constexpr int kBlockBytes = 18;  // 2-byte f16 scale + 16 sign bytes

// GEMV tiling: one LDS table serves a 512-column K tile; 64 rows per wave (one row per lane).
constexpr int kTileCols = 512;                       // 64 sign-byte positions
constexpr int kTilePos = kTileCols / 8;              // 64
constexpr int kRowBlock = 64;                        // rows per row-block (= lanes per wave)
constexpr int kUnitSignBytes = kRowBlock * kTilePos; // 4096 B of sign bytes per (row-block, tile)
constexpr int kUnitScaleBytes = kRowBlock * 4 * 2;   // 4 f16 scales per lane
constexpr int kUnitBytes = kUnitSignBytes + kUnitScaleBytes;  // 4608
constexpr int kLutBytes = 256 * kTilePos * 4;        // 64 KiB: f32 [256 sign-byte values][64 positions]

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));  // matrix-core accumulators

// DeltaNet state: [v-head][row i][column j] (row-major S[i][j]).  A thread holding 16 consecutive
// columns of one row moves them as four 16-byte words, so the 8 threads of a row cover 512
// contiguous bytes.  p is 16-byte aligned.
__device__ __forceinline__ void state_row_load(const float* p, float (&s)[16]) {
  const float4* q = reinterpret_cast<const float4*>(p);
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const float4 v = q[c];
    s[4 * c] = v.x;
    s[4 * c + 1] = v.y;
    s[4 * c + 2] = v.z;
    s[4 * c + 3] = v.w;
  }
}
__device__ __forceinline__ void state_row_store(float* p, const float (&s)[16]) {
  float4* q = reinterpret_cast<float4*>(p);
#pragma unroll
  for (int c = 0; c < 4; ++c) q[c] = make_float4(s[4 * c], s[4 * c + 1], s[4 * c + 2], s[4 * c + 3]);
}

// Device copy of one Q1_0 matrix in the GEMV layout.
//   unit (rb, t) at byte offset (rb * T + t) * kUnitBytes:
//     [chunk c 0..3][lane L 0..63][16 B]  stored sign byte s = 16c + i of lane L is the original
//                                          sign byte at tile position p = L ^ s
//     [lane L][4 x f16]                    scale slot j of lane L is tile group (L >> 4) ^ j
//   Row r = 64 rb + L; tile position p = 16 * (group within tile) + (byte within group).
struct Q1Dev {
  uint8_t* data = nullptr;
  int64_t rows = 0, cols = 0;  // logical shape
  int64_t nrb = 0;             // row-blocks (rows padded to 64)
  int64_t ntiles = 0;          // K tiles (cols padded to 512)
};

// p[0] + p[s] + p[2s] + ... + p[(n-1)s] (n >= 1), added in index order, with the loads issued 16 at a
// time: a loop of dependent adds with a run-time count otherwise waits one memory round trip per term.
// Every load of a round is issued (a term past n reloads term n-1, whose value is not added), so
// that no load sits behind a branch: predicated loads compile to branches whose merges wait for
// the loads already issued, and the round trips add up again.
__device__ __forceinline__ float ordered_sum(const float* __restrict__ p, int64_t stride, int n) {
  float v[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) v[k] = p[(size_t)min(k, n - 1) * stride];
  float acc = v[0];
#pragma unroll
  for (int k = 1; k < 16; ++k) acc = k < n ? acc + v[k] : acc;
  for (int b = 16; b < n; b += 16) {
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = p[(size_t)min(b + k, n - 1) * stride];
#pragma unroll
    for (int k = 0; k < 16; ++k) acc = b + k < n ? acc + v[k] : acc;
  }
  return acc;
}

// 1/rms of token n from the per-split sums of squares of a normed raw product (splits in order).
__device__ __forceinline__ float split_inv_rms(const float* __restrict__ ssq, int ssq_ld, int splits, int n, int64_t K,
                                               float eps) {
  const float ss = ordered_sum(ssq + n, ssq_ld, splits);
  return 1.0f / sqrtf(ss / (float)K + eps);
}

}  // namespace dz

#define DZ_HIP_CHECK(expr)                                                     \
  do {                                                                         \
    hipError_t _e = (expr);                                                    \
    if (_e != hipSuccess) return dz::set_error(DZ_ERR_DEVICE, "%s failed: %s (%s:%d)", #expr, hipGetErrorString(_e), __FILE__, __LINE__); \
  } while (0)

namespace dz {
int set_error(int code, const char* fmt, ...);
}
