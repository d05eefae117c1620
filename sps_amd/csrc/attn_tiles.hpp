// Cooperative global -> LDS staging of 32-row tiles and the per-element mask evaluation shared by
// the compute kernels and the mask-dump kernels.
#pragma once
#include "attn_kernels.hpp"
#include "cdna4.hpp"

namespace sps {

// LDS tile geometry. Rows are padded by 16 bytes so that the 32 rows read by one MFMA fragment
// land on distinct bank groups. Head dims below 32 are zero-padded to one 32-wide d chunk so the
// 32x32 MFMA shapes apply unchanged (the pad columns are zeroed once per kernel).
template <int D>
struct TileGeom {
  static constexpr int DC = (D + 31) / 32;               // 32-wide d chunks
  static constexpr int DPAD = DC * 32;
  static constexpr int RS = DPAD + 8;                    // LDS row stride (elements)
  static constexpr int CPR = D / 8;                      // 16-byte chunks per row
  static constexpr int RPP = 256 / CPR;                  // rows per pass of 256 threads
  static constexpr int PASSES = (kBlock + RPP - 1) / RPP;
  static constexpr int ELEMS = kBlock * RS;              // one staged tile
};

// Zeroes the pad columns [D, DPAD) of a staged tile (no-op for D >= 32).
template <int D>
__device__ __forceinline__ void zero_pad_cols(uint16_t* tile, int tid) {
  using G = TileGeom<D>;
  if constexpr (G::DPAD > D) {
    constexpr int per_row = (G::DPAD - D) / 8;
    for (int i = tid; i < kBlock * per_row; i += 256) {
      const int r = i / per_row, ch = i % per_row;
      u32x4_t z = {0u, 0u, 0u, 0u};
      lds_write_b128(tile + r * G::RS + D + ch * 8, z);
    }
  }
}

// Register staging for one 32-row tile of a [B, H, N, D] tensor. Row r of the tile is sequence
// position pos(r); rows at positions >= N are zero-filled.
template <int D>
struct TileRegs {
  u32x4_t v[TileGeom<D>::PASSES];

  template <class PosFn>
  __device__ __forceinline__ void load(const uint16_t* base, int64_t sn, int N, int tid, PosFn pos) {
    using G = TileGeom<D>;
#pragma unroll
    for (int p = 0; p < G::PASSES; ++p) {
      const int r = p * G::RPP + tid / G::CPR;
      const int ch = tid % G::CPR;
      u32x4_t x = {0u, 0u, 0u, 0u};
      if (r < kBlock) {
        const int kp = pos(r);
        if (kp < N) x = *reinterpret_cast<const u32x4_t*>(base + (int64_t)kp * sn + ch * 8);
      }
      v[p] = x;
    }
  }

  __device__ __forceinline__ void store(uint16_t* tile, int tid) const {
    using G = TileGeom<D>;
#pragma unroll
    for (int p = 0; p < G::PASSES; ++p) {
      const int r = p * G::RPP + tid / G::CPR;
      const int ch = tid % G::CPR;
      if (r < kBlock) lds_write_b128(tile + r * G::RS + ch * 8, v[p]);
    }
  }
};

// Query-stationary accumulator layout (S^T = K Q^T): the lane owns query `qp`, element i holds
// key row acc_row(i, g) of the key run. Returns bit i set when that pair is visible.
__device__ __forceinline__ uint32_t qs_mask_bits(const MaskSpec& m, int qp, int64_t dq, const KeyRun& kr,
                                                 int g, const int64_t* sdoc) {
  uint32_t bits = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int r = acc_row(i, g);
    const int kp = key_pos(m, kr, r);
    const int64_t dk = m.has_docs ? sdoc[r] : 0;
    bits |= (visible(m, qp, kp, dq, dk) ? 1u : 0u) << i;
  }
  return bits;
}

// Key-stationary accumulator layout (S = Q K^T): the lane owns key `kp`, element i holds query
// row acc_row(i, g) of the chunk starting at position qc.
__device__ __forceinline__ uint32_t ks_mask_bits(const MaskSpec& m, int qc, int kp, int64_t dk, int g,
                                                 const int64_t* sdoc) {
  uint32_t bits = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int r = acc_row(i, g);
    const int64_t dq = m.has_docs ? sdoc[r] : 0;
    bits |= (visible(m, qc + r, kp, dq, dk) ? 1u : 0u) << i;
  }
  return bits;
}

// Document range of a key run (only meaningful when m.has_docs).
__device__ __forceinline__ DocRange run_docs(const MaskSpec& m, const KeyRun& kr, const int64_t* gmin,
                                             const int64_t* gmax) {
  DocRange r = {0, 0};
  if (!m.has_docs) return r;
  int lo, hi;
  run_span(m, kr, lo, hi);
  return doc_range(gmin, gmax, lo, hi);
}

// Next key block after `i` of a query-stationary schedule that the workgroup's queries
// [qa, wg_qhi] cannot skip; returns s.n0 + s.n1 when none is left.
__device__ __forceinline__ int qs_next_block(const MaskSpec& m, const QSchedule& s, int qa, int wg_qhi,
                                             DocRange wg_qd, const int64_t* gmin, const int64_t* gmax,
                                             int i) {
  const int nb = s.n0 + s.n1;
  for (++i; i < nb; ++i) {
    const KeyRun kr = qschedule_block(s, i);
    if (classify(m, qa, wg_qhi, kr, wg_qd, run_docs(m, kr, gmin, gmax)) != TILE_SKIP) break;
  }
  return i;
}

// Next query chunk after `c` of a key-stationary schedule that the workgroup's key run cannot skip;
// returns s.c0 + s.nc when none is left.
__device__ __forceinline__ int ks_next_chunk(const MaskSpec& m, const KSchedule& s, const KeyRun& kr,
                                             DocRange kd, const int64_t* gmin, const int64_t* gmax, int c) {
  const int ce = s.c0 + s.nc;
  for (++c; c < ce; ++c) {
    const int qlo = c * kBlock;
    const int qhi = qlo + kBlock - 1 < m.N - 1 ? qlo + kBlock - 1 : m.N - 1;
    DocRange qd = {0, 0};
    if (m.has_docs) qd = doc_range(gmin, gmax, qlo, qhi);
    if (classify(m, qlo, qhi, kr, qd, kd) != TILE_SKIP) break;
  }
  return c;
}

}  // namespace sps
