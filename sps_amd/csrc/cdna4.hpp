// CDNA4 (gfx950) building blocks shared by the attention and decode kernels.
//
// Everything here is written for 64-lane wavefronts and the gfx950 matrix core:
//   * v_mfma_f32_32x32x16_{bf16,f16}: A is 32x16 (lane l holds row l%32, k = 8*(l/32)+j),
//     B is 16x32 (lane l holds column l%32, k = 8*(l/32)+j), C/D is 32x32 with lane l holding
//     column l%32 and rows 8*(i/4) + 4*(l/32) + (i%4) for i = 0..15.
//   * ds_read_b64_tr_b16: inside each 16-lane group, source lane s addresses row s/4 and
//     columns 4*(s%4)..+3 of a row-major 16-bit tile; result lane i receives the 4 rows of
//     column i. This reads K-contiguous MFMA fragments out of row-major LDS tiles, so no tile
//     is ever transposed on its way into LDS.
//   * v_permlane32_swap: exchanges the two 32-lane halves in one VALU op (cross-half reductions).
// The lane layouts above were checked on an MI355X with an in-bounds probe.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sps {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

#define SPS_LDS __attribute__((address_space(3)))

constexpr int kWave = 64;

// ---------------------------------------------------------------------------------------------
// Element types. Tiles are moved around as raw 16-bit words (u32x4 = 8 elements); only the MFMA
// and the fp32 <-> 16-bit conversions know the actual format.
// ---------------------------------------------------------------------------------------------
struct ElemBF16 {
  static __device__ __forceinline__ f32x16_t mfma(u32x4_t a, u32x4_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
  // Round-to-nearest-even pack of two fp32 values (v_cvt_pk_bf16_f32).
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    f32x2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
  }
  static __device__ __forceinline__ float to_f32(uint16_t x) {
    return __builtin_bit_cast(float, (uint32_t)x << 16);
  }
  // acc + lo + hi of a packed pair (v_dot2_f32_bf16 against {1, 1}).
  static __device__ __forceinline__ float sum2(uint32_t pair, float acc) {
    const uint32_t ones = 0x3f803f80u;
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pair), __builtin_bit_cast(bf16x2_t, ones),
                                          acc, false);
  }
  // acc + a.lo * b.lo + a.hi * b.hi of two packed pairs (v_dot2_f32_bf16; the products are exact in fp32).
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), acc,
                                          false);
  }
};

struct ElemF16 {
  static __device__ __forceinline__ f32x16_t mfma(u32x4_t a, u32x4_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    f32x2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_t));
  }
  static __device__ __forceinline__ float to_f32(uint16_t x) {
    return (float)__builtin_bit_cast(_Float16, x);
  }
  // acc + lo + hi of a packed pair (v_dot2_f32_f16 against {1, 1}).
  static __device__ __forceinline__ float sum2(uint32_t pair, float acc) {
    const uint32_t ones = 0x3c003c00u;
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, pair), __builtin_bit_cast(f16x2_t, ones), acc, false);
  }
  // acc + a.lo * b.lo + a.hi * b.hi of two packed pairs (v_dot2_f32_f16; the products are exact in fp32).
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b), acc, false);
  }
};

// ---------------------------------------------------------------------------------------------
// LDS access helpers.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ u32x4_t lds_read_b128(const uint16_t* p) {
  return *reinterpret_cast<const SPS_LDS u32x4_t*>(
      (const SPS_LDS uint16_t*)(p));
}

__device__ __forceinline__ void lds_write_b128(uint16_t* p, u32x4_t v) {
  *reinterpret_cast<SPS_LDS u32x4_t*>((SPS_LDS uint16_t*)(p)) = v;
}

// ds_read_b64_tr_b16 on a row-major 16-bit LDS tile: returns 4 consecutive rows of one column
// (see the header comment for the lane mapping).
__device__ __forceinline__ u32x2_t lds_read_tr16(const uint16_t* p) {
  i16x4_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((SPS_LDS i16x4_t*)((SPS_LDS uint16_t*)(p)));
  return __builtin_bit_cast(u32x2_t, r);
}

// Transposed 8-element MFMA fragment (K = rows of the LDS tile, M or N = columns).
// `tile` is a row-major [rows][row_stride] tile. For lane l the fragment holds column
// col0 + 16*((l/16)%2) + l%16 at rows r0 + 4*(l/32) + {0,1,2,3} and r0 + 8 + 4*(l/32) + {0,1,2,3}.
// This is exactly the K-order produced by a 32x32 MFMA accumulator (rows 8*(i/4)+4*(l/32)+i%4),
// so an accumulator converted to 16-bit pairs can be used directly as the other operand.
__device__ __forceinline__ u32x4_t lds_frag_tr(const uint16_t* tile, int row_stride, int r0, int col0,
                                               int lane) {
  const int s = lane & 15;
  const int grp = lane >> 4;
  const int row = r0 + 4 * (grp >> 1) + (s >> 2);
  const int col = col0 + 16 * (grp & 1) + 4 * (s & 3);
  u32x2_t lo = lds_read_tr16(tile + row * row_stride + col);
  u32x2_t hi = lds_read_tr16(tile + (row + 8) * row_stride + col);
  u32x4_t r = {lo[0], lo[1], hi[0], hi[1]};
  return r;
}

// ---------------------------------------------------------------------------------------------
// Cross-lane helpers.
// ---------------------------------------------------------------------------------------------
// permlane32_swap(u, u) returns {own, partner} on lanes 0-31 and {partner, own} on lanes 32-63,
// so symmetric reductions over the pair (l, l^32) need no lane id.
__device__ __forceinline__ float half_max(float x) {
  uint32_t u = __builtin_bit_cast(uint32_t, x);
  auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_elementwise_maximum(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
}

__device__ __forceinline__ float half_sum(float x) {
  uint32_t u = __builtin_bit_cast(uint32_t, x);
  auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ bool wave_any(bool p) { return __builtin_amdgcn_ballot_w64(p) != 0; }

// Raw buffer access: a descriptor over `bytes` bytes from `base`; loads at offsets >= bytes return
// zeros (the hardware range check), so tiles that run past the end of a sequence need no clamping.
typedef __amdgpu_buffer_rsrc_t BufRsrc;

// The base and size must be wave-uniform; they are moved to scalar registers explicitly, because a
// descriptor the compiler cannot prove uniform is kept in VGPRs and every load through it becomes a
// readfirstlane loop.
__device__ __forceinline__ BufRsrc make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t x = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(x >> 32));
  void* p = reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(p, (short)0, (int)__builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}

__device__ __forceinline__ u32x4_t buf_load_b128(BufRsrc r, uint32_t offset) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, 0);
}

// Direct global -> LDS loads (buffer_load ... lds): lane l's 16 (or 4) bytes at byte `voffset` of
// the buffer land at lds + 16 l (4 l), so one instruction fills a contiguous 1 KiB (256 B) block
// whose wave-uniform base goes to M0. The data never passes through VGPRs; completion is counted by
// vmcnt, so a wave waits for vmcnt before the barrier that hands the block to the other waves.
// Offsets past the descriptor's range load zeros, as for register loads.
__device__ __forceinline__ void lds_dma_b128(BufRsrc r, uint16_t* lds, uint32_t voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (SPS_LDS void*)((SPS_LDS uint16_t*)lds), 16, voffset, 0, 0, 0);
}

__device__ __forceinline__ void lds_dma_b32(BufRsrc r, float* lds, uint32_t voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (SPS_LDS void*)((SPS_LDS float*)lds), 4, voffset, 0, 0, 0);
}

// s_waitcnt vmcnt(0): waits for every outstanding vector-memory load of the wave. Placed before a
// software-pipelined loop so the compiler's wait counting does not fall back to vmcnt(0) inside it
// for registers loaded before the loop.
__device__ __forceinline__ void vmem_wait_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Reads a value that is uniform across the wave into a scalar register.
__device__ __forceinline__ int wave_uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

}  // namespace sps
