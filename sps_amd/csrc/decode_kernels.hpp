// Argument block, geometry and host launcher of the segmented decode kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sps {

constexpr int kMaxDecodeSegs = 3;
constexpr int kMaxDecodeExtras = 2;

// Work geometry for head dim D and K/V element size (bytes): each lane issues PASS 16-byte loads
// of K and of V; a workgroup of 4 waves covers CHUNK keys of one segment.
template <int D, int BYTES>
struct DecodeGeom {
  static constexpr int EPL = 16 / BYTES;
  static constexpr int LPR = D / EPL;
  static constexpr int RPP = 64 / LPR;
  static constexpr int PASS = 8;
  static constexpr int CHUNK = 4 * RPP * PASS;
  static constexpr int REC = D + 4;  // floats per partial record: acc[D], m, l, 2 pad
};

// Host-side helper with the same numbers (the kernels static_assert agreement).
inline int decode_chunk_keys(int D, int kv_bytes) { return 4 * (64 / (D / (16 / kv_bytes))) * 8; }
inline int decode_record_floats(int D) { return D + 4; }

struct DecodeSeg {
  const void* k;
  const void* v;
  int64_t ksb, ksh, kst;  // element strides of K (d stride 1)
  int64_t vsb, vsh, vst;  // element strides of V
  const void* len;        // [B] (shared by heads) or [B, H] live lengths, int32 or int64
  int len_i64;
  int len_per_head;
  int scan;               // scan length: keys t >= scan are never read
  int chunk_base;         // first chunk index of this segment
};

struct DecodeArgs {
  int B, H, NQ, n_seg, n_extra;
  DecodeSeg seg[kMaxDecodeSegs];
  const void* q;  // [B, nq, H, D] of q_dtype (values in the attention dtype), strides (b, slot, h)
  int q_dtype;    // 0 bf16, 1 f16, 2 f32
  int64_t q_sb, q_ss, q_sh;
  const void* ek[kMaxDecodeExtras];  // extra keys/values [B, H, D] of e_dtype, strides (b, h)
  const void* ev[kMaxDecodeExtras];
  int e_dtype;
  int64_t e_sb, e_sh;
  int emask[kMaxDecodeExtras];  // bit s: query slot s attends this extra
  float scale2;                 // sm_scale * log2(e)
  float* part;                  // workspace: [B*H, n_chunks, NQ, REC] partials
  int n_chunks;
  int chunk_keys;
  float* out;  // fp32, strides (b, slot, h), d stride 1
  int64_t o_sb, o_ss, o_sh;
};

// Element i of a bf16 / f16 / f32 array as fp32.
__device__ __forceinline__ float load_as_f32(const void* p, int64_t i, int dtype) {
  if (dtype == 2) return reinterpret_cast<const float*>(p)[i];
  const uint16_t x = reinterpret_cast<const uint16_t*>(p)[i];
  if (dtype == 1) return (float)__builtin_bit_cast(_Float16, x);
  return __builtin_bit_cast(float, (uint32_t)x << 16);
}

hipError_t launch_decode(const DecodeArgs& a, int D, int kv_dtype, hipStream_t stream);

}  // namespace sps
