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
  const float* q;  // fp32 (already rounded to the attention dtype), strides (b, slot, h), d stride 1
  int64_t q_sb, q_ss, q_sh;
  const float* ek[kMaxDecodeExtras];  // fp32 extra keys/values [B, H, D], strides (b, h)
  const float* ev[kMaxDecodeExtras];
  int64_t e_sb, e_sh;
  int emask[kMaxDecodeExtras];  // bit s: query slot s attends this extra
  float scale2;                 // sm_scale * log2(e)
  float* part;                  // workspace: [B*H, n_chunks, NQ, REC] partials
  int n_chunks;
  int chunk_keys;
  float* out;  // fp32, strides (b, slot, h), d stride 1
  int64_t o_sb, o_ss, o_sh;
};

hipError_t launch_decode(const DecodeArgs& a, int D, int kv_dtype, hipStream_t stream);

}  // namespace sps
