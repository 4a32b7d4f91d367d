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
// Loads are unconditional: an absent row reads a known-valid fallback
// address and is zeroed by a select when the registers go to LDS.  Keeping
// branches off the load path lets every load of a tile stay in flight while
// the previous tile is computed (a branch around a load forces the compiler
// to drain the memory counter at the join).
#pragma once

#include "fa_common.hpp"

namespace fa {

// x if keep else 0, component-wise (a whole-struct select defeats register
// promotion of the staging arrays).
__device__ inline uint4 masked(const uint4& x, uint32_t keep) {
  const uint32_t m = 0u - keep;
  return make_uint4(x.x & m, x.y & m, x.z & m, x.w & m);
}

template <typename Tag, int R, int COLS, int NT>
struct RowTile {
  using EL = Elem<Tag>;
  using S = typename EL::S;
  static constexpr int CE = EL::CE;
  static constexpr int CPR = COLS / CE;  // chunks per row
  static constexpr int CH = R * CPR;
  static constexpr int PT = (CH + NT - 1) / NT;
  uint4 r[PT];
  uint32_t ok;

  // rowptr(row) returns the address of element 0 of that tile row, or nullptr
  // for a zero row; `fallback` is any readable row of the same tensor.
  template <typename RowPtr>
  __device__ inline void load(RowPtr rowptr, const S* fallback, int tid) {
    ok = 0;
#pragma unroll
    for (int j = 0; j < PT; ++j) {
      const int c = tid + NT * j;
      const S* p = (CH % NT == 0 || c < CH) ? rowptr(c / CPR) : nullptr;
      ok |= (p != nullptr ? 1u : 0u) << j;
      p = p ? p : fallback;
      r[j] = *reinterpret_cast<const uint4*>(p + (c % CPR) * CE);
    }
  }
  __device__ inline void store(S* lds, int LD, int tid) const {
#pragma unroll
    for (int j = 0; j < PT; ++j) {
      const int c = tid + NT * j;
      if (CH % NT == 0 || c < CH)
        *reinterpret_cast<uint4*>(lds + (c / CPR) * LD + (c % CPR) * CE) = masked(r[j], (ok >> j) & 1u);
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
  uint4 r[PT * 4];  // flat: (item j, row q) at 4*j + q
  uint32_t ok;

  template <typename RowPtr>
  __device__ inline void load(RowPtr rowptr, const S* fallback, int tid) {
    ok = 0;
#pragma unroll
    for (int j = 0; j < PT; ++j) {
      const int it = tid + NT * j;
      const bool in = ITEMS % NT == 0 || it < ITEMS;
      const int rq = it / CPR, cc = it % CPR;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const S* p = in ? rowptr(4 * rq + q) : nullptr;
        ok |= (p != nullptr ? 1u : 0u) << (4 * j + q);
        p = p ? p : fallback;
        r[4 * j + q] = *reinterpret_cast<const uint4*>(p + cc * CE);
      }
    }
  }
  __device__ inline void store(S* lds, int LD, int tid) const {
#pragma unroll
    for (int j = 0; j < PT; ++j) {
      const int it = tid + NT * j;
      if (ITEMS % NT == 0 || it < ITEMS) {
        const int rq = it / CPR, cc = it % CPR;
        uint4 v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = masked(r[4 * j + q], (ok >> (4 * j + q)) & 1u);
        if constexpr (sizeof(S) == 2) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            // element e of each row sits in dword e/2, low half if e even
            const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
            uint2 w;
            w.x = __builtin_amdgcn_perm(word(v[1], e >> 1), word(v[0], e >> 1), sel);
            w.y = __builtin_amdgcn_perm(word(v[3], e >> 1), word(v[2], e >> 1), sel);
            *reinterpret_cast<uint2*>(lds + (cc * CE + e) * LD + 4 * rq) = w;
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            uint4 w = make_uint4(word(v[0], e), word(v[1], e), word(v[2], e), word(v[3], e));
            *reinterpret_cast<uint4*>(lds + (cc * CE + e) * LD + 4 * rq) = w;
          }
        }
      }
    }
  }

 private:
  __device__ static inline uint32_t word(const uint4& u, int k) {
    return k == 0 ? u.x : k == 1 ? u.y : k == 2 ? u.z : u.w;
  }
};

}  // namespace fa
