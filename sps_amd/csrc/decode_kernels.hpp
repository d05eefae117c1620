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
  static constexpr int PASS = 16;
  static constexpr int CHUNK = 4 * RPP * PASS;
  static constexpr int REC = D + 4;  // floats per partial record: acc[D], m, l, 2 pad
};

// Host-side helper with the same numbers (the kernels static_assert agreement).
inline int decode_chunk_keys(int D, int kv_bytes) { return 4 * (64 / (D / (16 / kv_bytes))) * 16; }
inline int decode_record_floats(int D) { return D + 4; }

// Decode KV-cache update of one layer: ring (normal window) insert + retained append.
constexpr int kMaxVecHeads = 1024;  // heads per sequence the 16-byte path keeps in LDS

struct KvUpdateArgs {
  int B, H, D;
  int kv_dtype;   // cache element type: 0 bf16, 1 f16, 2 f32
  int new_dtype;  // new K/V element type (converted to kv_dtype, round to nearest even)
  // Ring: K/V [B, H, storage, D] (strides b, h, t); len and pos [B]; window <= 0 leaves it untouched.
  void* ring_k;
  void* ring_v;
  int64_t rk_sb, rk_sh, rk_st, rv_sb, rv_sh, rv_st;
  int ring_storage, window;
  void* ring_len;
  void* ring_pos;
  int64_t ring_len_sb, ring_pos_sb;
  // Retained: K/V [B, H, storage, D]; len [B, H].
  void* ret_k;
  void* ret_v;
  int64_t tk_sb, tk_sh, tk_st, tv_sb, tv_sh, tv_st;
  int ret_storage;
  void* ret_len;
  int64_t ret_len_sb, ret_len_sh;
  int len_i64;  // lengths and positions: int64 (else int32)
  // New K/V [B, H, D] (strides b, h) for the ring slot and the retained slot.
  const void* kw;
  const void* vw;
  const void* kr;
  const void* vr;
  int64_t kw_sb, kw_sh, vw_sb, vw_sh, kr_sb, kr_sh, vr_sb, vr_sh;
  const void* active;  // [B]: nonzero = update this sequence
  int active_bytes;    // 1, 4 or 8
  int64_t active_sb;
  int vec16;  // same dtype, rows and strides 16-byte aligned, H <= kMaxVecHeads: 16-byte pieces
};

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
  int q_packed;   // q has the K/V's 16-bit dtype, a 16-byte aligned base and strides of 8k elements
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
  // KV update folded into the launch (sps_decode_kv_update), when snap is not null: the partial
  // kernel's first-chunk workgroup of each (b, h) stores the lengths both kernels use into
  // snap[(b H + h) kSnapWords ...]: the live length of each segment, then the update's old ring
  // length, ring position, retained length and active flag. The merge kernel reads only these, so
  // it can write the new rows and advance the lengths in the same launch.
  int64_t* snap;
  KvUpdateArgs upd;
};

constexpr int kSnapWords = 8;  // int64 words per (b, h): 3 segment lengths, ring len, ring pos, retained len, active
constexpr int kSnapRingLen = kMaxDecodeSegs, kSnapRingPos = kMaxDecodeSegs + 1, kSnapRetLen = kMaxDecodeSegs + 2,
              kSnapActive = kMaxDecodeSegs + 3;

// Element i of a bf16 / f16 / f32 array as fp32.
__device__ __forceinline__ float load_as_f32(const void* p, int64_t i, int dtype) {
  if (dtype == 2) return reinterpret_cast<const float*>(p)[i];
  const uint16_t x = reinterpret_cast<const uint16_t*>(p)[i];
  if (dtype == 1) return (float)__builtin_bit_cast(_Float16, x);
  return __builtin_bit_cast(float, (uint32_t)x << 16);
}

// Lengths and positions (int32 or int64) and active flags (1, 4 or 8 bytes) of the KV caches.
__device__ __forceinline__ int64_t cache_len_load(const void* p, int64_t i, int i64) {
  return i64 ? reinterpret_cast<const int64_t*>(p)[i] : (int64_t) reinterpret_cast<const int*>(p)[i];
}
__device__ __forceinline__ void cache_len_store(void* p, int64_t i, int i64, int64_t v) {
  if (i64)
    reinterpret_cast<int64_t*>(p)[i] = v;
  else
    reinterpret_cast<int*>(p)[i] = (int)v;
}
__device__ __forceinline__ bool cache_flag_load(const void* p, int64_t i, int bytes) {
  if (bytes == 1) return reinterpret_cast<const uint8_t*>(p)[i] != 0;
  if (bytes == 4) return reinterpret_cast<const int*>(p)[i] != 0;
  return reinterpret_cast<const int64_t*>(p)[i] != 0;
}

hipError_t launch_decode(const DecodeArgs& a, int D, int kv_dtype, hipStream_t stream);

hipError_t launch_kv_update(const KvUpdateArgs& a, hipStream_t stream);

// Pre-attention rotary embedding of Q and K and cast of Q, K, V (one pass; rope.hip).
struct RopeArgs {
  int B, N, H, D;
  int in_dtype, out_dtype;  // 0 bf16, 1 f16, 2 f32
  const void* q;
  const void* k;
  const void* v;
  int64_t q_sb, q_sn, q_sh, k_sb, k_sn, k_sh, v_sb, v_sn, v_sh;
  const float* freqs;  // real view of complex64 freqs: [.., N, D/2, 2]
  int64_t f_sb, f_sn;  // float strides (f_sb = 0: shared by all sequences)
  void* qo;
  void* ko;
  void* vo;
  int64_t qo_sb, qo_sn, qo_sh, ko_sb, ko_sn, ko_sh, vo_sb, vo_sn, vo_sh;
};
hipError_t launch_rope_qkv(const RopeArgs& a, hipStream_t stream);

// Prefill -> decode caches of one layer (prefill_state.hip).
struct PrefillStateArgs {
  int B, T, H, D;
  int in_dtype, kv_dtype;
  const void* k;  // [B, 2T, H, D] (strides b, n, h)
  const void* v;
  int64_t k_sb, k_sn, k_sh, v_sb, v_sn, v_sh;
  int window_slot, retained_slot;  // parity of the ring / retained rows in the 2T positions
  const uint8_t* mask;             // [B, T] current-document tokens (nonzero = member)
  int64_t mask_sb;
  void* ring_k;
  void* ring_v;
  int64_t rk_sb, rk_sh, rk_st, rv_sb, rv_sh, rv_st;
  int ring_storage, window;
  void* ring_len;
  void* ring_pos;
  int64_t ring_len_sb, ring_pos_sb;
  void* ret_k;
  void* ret_v;
  int64_t tk_sb, tk_sh, tk_st, tv_sb, tv_sh, tv_st;
  int ret_storage;
  void* ret_len;
  int64_t ret_len_sb, ret_len_sh;
  int len_i64;
};
hipError_t launch_prefill_state(const PrefillStateArgs& a, hipStream_t stream);

}  // namespace sps
