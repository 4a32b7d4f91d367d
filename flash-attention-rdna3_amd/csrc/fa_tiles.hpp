// fa_tiles.hpp - global -> register -> LDS staging of K/V/Q/dO tiles.
//
// Tiles are moved in 16-byte chunks so every global access is a coalesced
// dwordx4 load: consecutive threads read consecutive chunks of one row.  Rows
// past the valid range are zero-filled (a zero V row keeps 0 * garbage out of
// the P.V product).  Two LDS layouts exist:
//   RowTile   : T[row][col]   (row stride LD), read as MFMA operands with the
//               contracted index along col.
//   TransTile : T[col][row]   (row stride LD), i.e. the tile transposed, read
//               when the contracted index is the tile's row (P.V, dS^T.Q ...).
//               Each thread loads 4 consecutive rows of one chunk and writes
//               4-row runs, so LDS writes are 8 (16-bit) or 16 (fp32) bytes.
#pragma once

#include "fa_common.hpp"

namespace fa {

template <typename Tag, int R, int COLS, int NT>
struct RowTile {
  using EL = Elem<Tag>;
  using S = typename EL::S;
  static constexpr int CE = EL::CE;
  static constexpr int CPR = COLS / CE;  // chunks per row
  static constexpr int CH = R * CPR;
  static constexpr int PT = (CH + NT - 1) / NT;
  uint4 r[PT];

  // rowptr(row) returns the address of element 0 of that tile row, or nullptr
  // for a zero row.
  template <typename RowPtr>
  __device__ inline void load(RowPtr rowptr, int tid) {
#pragma unroll
    for (int j = 0; j < PT; ++j) {
      const int c = tid + NT * j;
      r[j] = make_uint4(0u, 0u, 0u, 0u);
      if (CH % NT == 0 || c < CH) {
        const S* p = rowptr(c / CPR);
        if (p) r[j] = *reinterpret_cast<const uint4*>(p + (c % CPR) * CE);
      }
    }
  }
  __device__ inline void store(S* lds, int LD, int tid) const {
#pragma unroll
    for (int j = 0; j < PT; ++j) {
      const int c = tid + NT * j;
      if (CH % NT == 0 || c < CH)
        *reinterpret_cast<uint4*>(lds + (c / CPR) * LD + (c % CPR) * CE) = r[j];
    }
  }
};

template <typename Tag, int R, int COLS, int NT>
struct TransTile {
  using EL = Elem<Tag>;
  using S = typename EL::S;
  static constexpr int CE = EL::CE;
  static constexpr int CPR = COLS / CE;
  static constexpr int ITEMS = (R / 4) * CPR;  // (row quad, chunk)
  static constexpr int PT = (ITEMS + NT - 1) / NT;
  uint4 r[PT][4];

  template <typename RowPtr>
  __device__ inline void load(RowPtr rowptr, int tid) {
#pragma unroll
    for (int j = 0; j < PT; ++j) {
      const int it = tid + NT * j;
#pragma unroll
      for (int q = 0; q < 4; ++q) r[j][q] = make_uint4(0u, 0u, 0u, 0u);
      if (ITEMS % NT == 0 || it < ITEMS) {
        const int rq = it / CPR, cc = it % CPR;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const S* p = rowptr(4 * rq + q);
          if (p) r[j][q] = *reinterpret_cast<const uint4*>(p + cc * CE);
        }
      }
    }
  }
  __device__ inline void store(S* lds, int LD, int tid) const {
#pragma unroll
    for (int j = 0; j < PT; ++j) {
      const int it = tid + NT * j;
      if (ITEMS % NT == 0 || it < ITEMS) {
        const int rq = it / CPR, cc = it % CPR;
        if constexpr (sizeof(S) == 2) {
          const uint16_t* v0 = reinterpret_cast<const uint16_t*>(&r[j][0]);
          const uint16_t* v1 = reinterpret_cast<const uint16_t*>(&r[j][1]);
          const uint16_t* v2 = reinterpret_cast<const uint16_t*>(&r[j][2]);
          const uint16_t* v3 = reinterpret_cast<const uint16_t*>(&r[j][3]);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            uint2 w;
            w.x = (uint32_t)v0[e] | ((uint32_t)v1[e] << 16);
            w.y = (uint32_t)v2[e] | ((uint32_t)v3[e] << 16);
            *reinterpret_cast<uint2*>(lds + (cc * CE + e) * LD + 4 * rq) = w;
          }
        } else {
          const uint32_t* v0 = reinterpret_cast<const uint32_t*>(&r[j][0]);
          const uint32_t* v1 = reinterpret_cast<const uint32_t*>(&r[j][1]);
          const uint32_t* v2 = reinterpret_cast<const uint32_t*>(&r[j][2]);
          const uint32_t* v3 = reinterpret_cast<const uint32_t*>(&r[j][3]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            uint4 w = make_uint4(v0[e], v1[e], v2[e], v3[e]);
            *reinterpret_cast<uint4*>(lds + (cc * CE + e) * LD + 4 * rq) = w;
          }
        }
      }
    }
  }
};

}  // namespace fa
