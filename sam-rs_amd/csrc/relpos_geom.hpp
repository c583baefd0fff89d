// Key-tile geometry shared by the rel-pos attention kernels (f16/bf16 and f32).
//
// A key tile holds 64 "slots" that cover whole rows of the H x W key grid: 4 rows padded to 16 columns
// (W <= 16), 2 rows padded to 32 (W <= 32), or 1 row padded to 64 (W <= 64). With 32x32 MFMA tiles a
// lane holds the scores of one query for 16 slots per 32-slot block, always at the same grid columns,
// which is what lets the Rw part of the bias stay in registers for the whole key loop.
#pragma once
#include "common.hpp"

namespace samhip {

enum KeyMode { kPair = 0, kRow32 = 1, kRow64 = 2 };

template <int MODE> struct KeyGeom {
  static constexpr int RPT = MODE == kPair ? 4 : (MODE == kRow32 ? 2 : 1);  // grid rows per tile
  static constexpr int WP = MODE == kPair ? 16 : (MODE == kRow32 ? 32 : 64);  // padded row width
  static constexpr int RWN = MODE == kRow64 ? 32 : 16;                        // Rw registers per lane
  // Slot (0..63) of S^T row m (0..31) of 32-key block mb. m = 4*h + 8*a + b as the MFMA lays it out.
  __device__ static __forceinline__ int slot(int mb, int m) {
    if (MODE == kPair) {
      const int h = (m >> 2) & 1, a = m >> 3, b = m & 3;
      return 32 * mb + 16 * h + 4 * a + b;  // grid row 2*mb + h, column 4*a + b
    }
    return 32 * mb + m;
  }
  // Grid row (within the tile) of 32-key block mb for lane half h.
  __device__ static __forceinline__ int row(int mb, int h) {
    if (MODE == kPair) return 2 * mb + h;
    if (MODE == kRow32) return mb;
    return 0;
  }
  // Column of accumulator element e (m = 8*(e/4) + 4*h + e%4) in block mb.
  __device__ static __forceinline__ int col(int mb, int e, int h) {
    const int a = e >> 2, b = e & 3;
    if (MODE == kPair) return 4 * a + b;
    if (MODE == kRow32) return 4 * h + 8 * a + b;
    return 32 * mb + 4 * h + 8 * a + b;
  }
  __device__ static __forceinline__ int rw_index(int mb, int e) { return MODE == kRow64 ? 16 * mb + e : e; }
};

constexpr float kLog2e = 1.4426950408889634f;

}  // namespace samhip
