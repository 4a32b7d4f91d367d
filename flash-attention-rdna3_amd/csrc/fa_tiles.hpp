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

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Eight fp8 (OCP e4m3) cache elements -> an 8-element 16-bit operand of the
// query's type.  The conversion is exact (e4m3 values are representable in
// fp16 and bf16); the per-tensor scales are applied outside (k_scale in the
// logit scale, v_scale on the output).
template <typename Tag, bool HI>
__device__ inline uint32_t fp8x2_to_16(uint32_t w) {
  if constexpr (std::is_same<Tag, bf16_t>::value)
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w, 1.0f, HI));
  else
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)w, 1.0f, HI));
}
template <typename Tag>
__device__ inline s16x8 fp8x8_to_op(u32x2 r) {
  const uint32_t p[4] = {fp8x2_to_16<Tag, false>(r[0]), fp8x2_to_16<Tag, true>(r[0]),
                         fp8x2_to_16<Tag, false>(r[1]), fp8x2_to_16<Tag, true>(r[1])};
  s16x8 o;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[2 * i] = (short)(p[i] & 0xFFFFu);
    o[2 * i + 1] = (short)(p[i] >> 16);
  }
  return o;
}

// Eight fp8 cache elements at p (8-byte aligned) as one 16-byte chunk of
// 16-bit elements of the query's type.
template <typename Tag>
__device__ inline uint4 fp8_chunk(const uint8_t* p) {
  return __builtin_bit_cast(uint4, fp8x8_to_op<Tag>(*reinterpret_cast<const u32x2*>(p)));
}


// KV8: the rows hold fp8 (e4m3) elements, converted to Tag as they load.
template <typename Tag, int R, int COLS, int NT, bool KV8 = false>
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
  template <typename RowPtr, typename P>
  __device__ inline void load(RowPtr rowptr, const P* fallback, int tid) {
    ok = 0;
#pragma unroll
    for (int j = 0; j < PT; ++j) {
      const int c = tid + NT * j;
      const P* p = (CH % NT == 0 || c < CH) ? rowptr(c / CPR) : nullptr;
      ok |= (p != nullptr ? 1u : 0u) << j;
      p = p ? p : fallback;
      if constexpr (KV8) r[j] = fp8_chunk<Tag>(p + (c % CPR) * CE);
      else r[j] = *reinterpret_cast<const uint4*>(p + (c % CPR) * CE);
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

template <typename Tag, int R, int COLS, int NT, bool KV8 = false>
struct TransTile {
  using EL = Elem<Tag>;
  using S = typename EL::S;
  static constexpr int CE = EL::CE;
  static constexpr int CPR = COLS / CE;
  static constexpr int ITEMS = (R / 4) * CPR;  // (row quad, chunk)
  static constexpr int PT = (ITEMS + NT - 1) / NT;
  uint4 r[PT * 4];  // flat: (item j, row q) at 4*j + q
  uint32_t ok;

  template <typename RowPtr, typename P>
  __device__ inline void load(RowPtr rowptr, const P* fallback, int tid) {
    ok = 0;
#pragma unroll
    for (int j = 0; j < PT; ++j) {
      const int it = tid + NT * j;
      const bool in = ITEMS % NT == 0 || it < ITEMS;
      const int rq = it / CPR, cc = it % CPR;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const P* p = in ? rowptr(4 * rq + q) : nullptr;
        ok |= (p != nullptr ? 1u : 0u) << (4 * j + q);
        p = p ? p : fallback;
        if constexpr (KV8) r[4 * j + q] = fp8_chunk<Tag>(p + cc * CE);
        else r[4 * j + q] = *reinterpret_cast<const uint4*>(p + cc * CE);
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

namespace fa {

// ---------------------------------------------------------------------------
// Swizzled row-major LDS tiles for 16-bit data (no padding).
//
// A tile row of COLS elements is COLS/8 chunks of 16 bytes; chunk c of row r
// is stored at chunk slot c ^ swz(r).  swz is chosen per row width so that
// both read patterns the kernels use are bank-conflict free on the 64-bank
// LDS:
//  * ds_read_b128 of one chunk from 16 consecutive rows (MFMA operand with
//    the contracted index along the row), and
//  * ds_read_b64_tr_b16 over an aligned block of 4 rows x 4 chunks (MFMA
//    operand with the contracted index along the column; see tr_op_rowmap).
// ---------------------------------------------------------------------------
template <int COLS>
__device__ constexpr inline int swz(int r) {
  constexpr int CPR = COLS / 8;
  if constexpr (CPR >= 16) return ((r & 3) << 2) | ((r >> 2) & 3);
  else if constexpr (CPR == 8) return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
  else return (r >> 2) & 3;
}

template <int COLS>
__device__ constexpr inline int swz_off(int r, int col) {
  return r * COLS + (((col >> 3) ^ swz<COLS>(r)) << 3) + (col & 7);
}

template <int R, int COLS, int NT>
struct SwzTile {
  static constexpr int CPR = COLS / 8;
  static constexpr int CH = R * CPR;
  static constexpr int PT = (CH + NT - 1) / NT;
  uint4 r[PT];
  uint32_t ok;

  template <typename RowPtr>
  __device__ inline void load(RowPtr rowptr, const uint16_t* fallback, int tid) {
    ok = 0;
#pragma unroll
    for (int j = 0; j < PT; ++j) {
      const int c = tid + NT * j;
      const uint16_t* p = (CH % NT == 0 || c < CH) ? rowptr(c / CPR) : nullptr;
      ok |= (p != nullptr ? 1u : 0u) << j;
      p = p ? p : fallback;
      r[j] = *reinterpret_cast<const uint4*>(p + (c % CPR) * 8);
    }
  }
  __device__ inline void store(uint16_t* lds, int tid) const {
#pragma unroll
    for (int j = 0; j < PT; ++j) {
      const int c = tid + NT * j;
      if (CH % NT == 0 || c < CH) {
        const int row = c / CPR, ch = c % CPR;
        *reinterpret_cast<uint4*>(lds + row * COLS + ((ch ^ swz<COLS>(row)) << 3)) = masked(r[j], (ok >> j) & 1u);
      }
    }
  }
};

// B/A operand (8 x 16-bit) of row `row`, k-chunk `chunk` of a swizzled tile.
template <int COLS>
__device__ inline s16x8 swz_op(const uint16_t* tile, int row, int chunk) {
  return *reinterpret_cast<const s16x8*>(tile + row * COLS + ((chunk ^ swz<COLS>(row)) << 3));
}

// A operand for a product contracting over the TILE ROW index whose k-slots
// follow a 32x32 accumulator's row map (the layout pack_op produces): slot e
// of lane half h is tile row rbase + 32*(j/2) + 16*(j%2) + 8*(e/4) + 4h + e%4,
// operand row (lane%32) is tile column cbase + lane%32.  Two
// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element i%4
// of the 4-element chunks read by lanes 4e + i/4, so lane `src` of a group
// reads 4 columns at row (src/4) of the 4-row block and the result is the
// column of the block.
template <int COLS>
__device__ inline s16x8 tr_op_rowmap(const uint16_t* tile, int rbase, int cbase, int j, int lane) {
  const int h = lane >> 5;
  const int row0 = rbase + 32 * (j >> 1) + 16 * (j & 1) + 4 * h + ((lane & 15) >> 2);
  const int col = cbase + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  typedef short s4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s4 lds_s4;
  const s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_s4*)(const_cast<uint16_t*>(tile) + swz_off<COLS>(row0, col)));
  const s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_s4*)(const_cast<uint16_t*>(tile) + swz_off<COLS>(row0 + 8, col)));
  s16x8 r = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return r;
}

// ---------------------------------------------------------------------------
// Buffer-addressed tiles.  A buffer resource covers the valid rows of a tile
// window (its base is rebased per tile in scalar registers); every lane's
// byte offset inside the window is fixed, so a load is one buffer_load with a
// constant VGPR offset, and rows past the valid range read as zero from the
// hardware range check instead of a per-row test.  Offsets are 32-bit: the
// host only takes these paths when R * row stride * 2 bytes < 2^31.
// ---------------------------------------------------------------------------
template <int COLS>
__device__ inline __amdgpu_buffer_rsrc_t rows_rsrc(const uint16_t* row0, int64_t stride, int rows) {
  const uint32_t bytes = rows > 0 ? (uint32_t)((int64_t)(rows - 1) * stride * 2 + COLS * 2) : 0u;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(row0), (short)0, (int)bytes, 0x00020000);
}

template <int R, int COLS, int NT>
struct BufSwzTile {
  static constexpr int CPR = COLS / 8;
  static constexpr int CH = R * CPR;
  static constexpr int PT = (CH + NT - 1) / NT;
  uint32_t voff[PT];
  s16x8 r[PT];

  __device__ inline void init(int64_t stride, int tid) {
#pragma unroll
    for (int j = 0; j < PT; ++j) {
      const int c = tid + NT * j;
      const int row = c / CPR, ch = c % CPR;
      voff[j] = (CH % NT == 0 || c < CH) ? (uint32_t)(row * stride * 2 + ch * 16) : 0u;
    }
  }
  __device__ inline void load(__amdgpu_buffer_rsrc_t rs) {
#pragma unroll
    for (int j = 0; j < PT; ++j)
      r[j] = __builtin_bit_cast(s16x8, __builtin_amdgcn_raw_buffer_load_b128(rs, voff[j], 0, 0));
  }
  __device__ inline void store(uint16_t* lds, int tid) const {
#pragma unroll
    for (int j = 0; j < PT; ++j) {
      const int c = tid + NT * j;
      if (CH % NT == 0 || c < CH) {
        const int row = c / CPR, ch = c % CPR;
        *reinterpret_cast<s16x8*>(lds + row * COLS + ((ch ^ swz<COLS>(row)) << 3)) = r[j];
      }
    }
  }
};

// ---------------------------------------------------------------------------
// HBM -> LDS tiles without register staging: buffer_load_dwordx4 ... lds.
// Each instruction of a wave fills 1 KB of LDS contiguously (lane i at +16*i,
// base in M0); each lane picks the global 16-byte chunk whose swizzled LDS
// slot is its own, so the tile lands in the swz<COLS> layout.  The load is
// issued from inline asm: the compiler does not track it, so it neither
// drains it before unrelated LDS reads nor waits for it at all -- the kernel
// waits (vmcnt) and synchronises (barrier) before reading the tile.  The asm
// writes M0, which the compiler reserves (hence its -Winline-asm warning):
// no other instruction of these kernels reads M0 (no LDS-direct, movrel,
// GWS or message instructions; the generated code was checked), so nothing
// depends on a value the asm overwrites.
// ---------------------------------------------------------------------------
typedef int i32x4 __attribute__((ext_vector_type(4)));

__device__ inline i32x4 rsrc_words(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  r[1] = __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xFFFFu));
  r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
  r[3] = 0x00020000;
  return r;
}

template <int COLS>
__device__ inline i32x4 rows_rsrc_words(const uint16_t* row0, int64_t stride, int rows) {
  const uint32_t bytes = rows > 0 ? (uint32_t)((int64_t)(rows - 1) * stride * 2 + COLS * 2) : 0u;
  return rsrc_words(row0, bytes);
}

__device__ inline void buf_load_lds16(i32x4 rs, uint32_t voff, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(voff), "s"(rs), "s"(lds_addr)
               : "memory", "m0");
}

// The same load, nontemporal: the lines are not kept in L2 for reuse.
__device__ inline void buf_load_lds16_nt(i32x4 rs, uint32_t voff, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen nt lds"
               :
               : "v"(voff), "s"(rs), "s"(lds_addr)
               : "memory", "m0");
}

template <int R, int COLS, int NT>
struct DmaSwzTile {
  static constexpr int CPR = COLS / 8;
  static constexpr int CH = R * CPR;
  static_assert(CH % NT == 0, "tile must be a whole number of 16-byte chunks per thread");
  static constexpr int PT = CH / NT;
  uint32_t voff[PT];

  __device__ inline void init(int64_t stride, int tid) {
#pragma unroll
    for (int j = 0; j < PT; ++j) {
      const int slot = NT * j + tid;
      const int row = slot / CPR;
      const int lc = (slot % CPR) ^ swz<COLS>(row);
      voff[j] = (uint32_t)(row * stride * 2 + lc * 16);
    }
  }
  // Source tile stored as column blocks of SUB_CHUNKS 16-byte chunks: row r
  // of block k at k * block_bytes + r * SUB_CHUNKS * 16 (the LDS tile is the
  // same row-major swizzled tile as with init).
  template <int SUB_CHUNKS>
  __device__ inline void init_blocked(int block_bytes, int tid) {
#pragma unroll
    for (int j = 0; j < PT; ++j) {
      const int slot = NT * j + tid;
      const int row = slot / CPR;
      const int lc = (slot % CPR) ^ swz<COLS>(row);
      voff[j] = (uint32_t)((lc / SUB_CHUNKS) * block_bytes + row * SUB_CHUNKS * 16 + (lc % SUB_CHUNKS) * 16);
    }
  }
  // lds_tile: byte address of the tile in LDS; wave: this wave's index.
  __device__ inline void load(i32x4 rs, uint32_t lds_tile, int wave) const {
#pragma unroll
    for (int j = 0; j < PT; ++j) buf_load_lds16(rs, voff[j], lds_tile + (uint32_t)(NT * j + 64 * wave) * 16u);
  }
  __device__ inline void load_nt(i32x4 rs, uint32_t lds_tile, int wave) const {
#pragma unroll
    for (int j = 0; j < PT; ++j) buf_load_lds16_nt(rs, voff[j], lds_tile + (uint32_t)(NT * j + 64 * wave) * 16u);
  }
};

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding).
template <int N>
__device__ inline void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

__device__ inline uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Scheduling hint for a block of N MFMAs that each consume RPM LDS reads:
// issue the reads of the first AHEAD MFMAs first, then alternate one MFMA
// with the reads of a later one, so LDS latency overlaps MFMA execution
// instead of each MFMA waiting on its own reads.  (sched_group_barrier
// masks: 0x008 MFMA, 0x100 DS read.)
// EXTRA: further LDS reads at the head of the block (e.g. accumulator seeds).
template <int N, int AHEAD, int RPM = 1, int EXTRA = 0>
__device__ inline void sched_read_ahead() {
  constexpr int A = AHEAD < N ? AHEAD : N;
  __builtin_amdgcn_sched_group_barrier(0x100, A * RPM + EXTRA, 0);
#pragma unroll
  for (int i = 0; i < N - A; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, RPM, 0);
  }
  __builtin_amdgcn_sched_group_barrier(0x008, A, 0);
}


// A 32x32 fp32 accumulator (16 values per lane) parked in LDS and read back
// as four 16-byte chunks per lane, chunk-major (chunk c of lane L at float
// offset (64 * c + L) * 4), so every ds_write_b128 / ds_read_b128 of a wave
// covers 1 KiB of consecutive addresses.  A block takes 1024 floats.
__device__ inline void park_acc(float* blk, int lane, const f32x16& a) {
  f32x4* p = reinterpret_cast<f32x4*>(blk);
#pragma unroll
  for (int c = 0; c < 4; ++c) p[64 * c + lane] = f32x4{a[4 * c], a[4 * c + 1], a[4 * c + 2], a[4 * c + 3]};
}
__device__ inline f32x16 unpark_acc(const float* blk, int lane) {
  const f32x4* p = reinterpret_cast<const f32x4*>(blk);
  f32x16 a;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const f32x4 v = p[64 * c + lane];
    a[4 * c] = v[0];
    a[4 * c + 1] = v[1];
    a[4 * c + 2] = v[2];
    a[4 * c + 3] = v[3];
  }
  return a;
}

// Whole-row store of a wave's 32 x D 16-bit output held as 32x32 MFMA
// accumulators (lane%32 = row, acc[db][4g + r] = column 32 db + 8 g + 4 h + r,
// h = lane/32).  Written straight from that layout, every store instruction
// would put 8 bytes into each of 32 rows, i.e. partial 128-byte lines in
// HBM (twice the output bytes were written back).  Instead the rows go
// through LDS (kStageRowBytes per row, padded so the 32 lanes' writes of
// one column fall in distinct banks), then each lane stores 16 consecutive
// bytes and a wave instruction covers 64 x 16 bytes of whole rows.
// `stage` is this wave's LDS area of 32 * (D + 8) halfs (8.5 KiB at
// D = 128), not used by any other wave at this point; all 64 lanes must
// call (rows >= nrows are staged but not stored).
template <typename Tag, int D>
__device__ inline void store_rows_staged(const f32x16 (&acc)[D / 32], float scale, uint16_t* stage,
                                         uint16_t* out_row0, int64_t row_stride, int nrows, int lane) {
  using EL = Elem<Tag>;
  constexpr int RS = D + 8;  // staged row stride (halfs): 16-byte aligned rows
  const int h = lane >> 5, l32 = lane & 31;
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      s16x4 w;
#pragma unroll
      for (int r = 0; r < 4; ++r) w[r] = (short)EL::from_f(acc[db][4 * g + r] * scale);
      *reinterpret_cast<s16x4*>(stage + l32 * RS + db * 32 + 8 * g + 4 * h) = w;
    }
  // (a wave's LDS operations complete in issue order: the reads below see
  // every lane's writes above)
  constexpr int CPR = D / 8;       // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;    // rows per wave instruction
  const int rsub = lane / CPR, ch = lane % CPR;
#pragma unroll
  for (int i = 0; i < 32 / RPI; ++i) {
    const int row = i * RPI + rsub;
    const s16x8 v = *reinterpret_cast<const s16x8*>(stage + row * RS + ch * 8);
    if (row < nrows) *reinterpret_cast<s16x8*>(out_row0 + (int64_t)row * row_stride + ch * 8) = v;
  }
}

}  // namespace fa
