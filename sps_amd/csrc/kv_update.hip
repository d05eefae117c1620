// Decode KV-cache update of one layer in one launch: the current token's K/V go into the ring
// (normal-window) cache and are appended to the retained cache.
//
// Semantics (per sequence b with active[b] != 0), those of the reference's un-fused PyTorch path
// _update_normal_memory_unfused / _update_predict_memory_unfused (reverse_sps/inference.py:137-168,
// 240-268), with the fused kernel's retained bound check (utils/decode_attention_fast.py:95-104):
//   ring (window > 0): slot = len[b] >= window ? pos[b] : len[b]; K/V[b, h, slot] = new (every h);
//     then len[b] += 1 while the ring fills, else pos[b] = (pos[b] + 1) % window.
//   retained: if 0 <= len[b, h] < storage: K/V[b, h, len[b, h]] = new, len[b, h] += 1.
// One workgroup per sequence reads the old lengths, writes every head's rows, and only then (after
// a barrier) advances the lengths, so no head ever sees a half-updated ring position. (The
// reference's fused kernel advances len/pos from the head-0 program while other heads' programs may
// still be reading them.)
#include "cdna4.hpp"
#include "decode_kernels.hpp"

namespace sps {

namespace {

// Copies element `src_i` of `src` (src_dtype) to element `dst_i` of `dst` (dst_dtype). Equal types
// copy the bits; otherwise through fp32 with round-to-nearest-even (what torch's .to() does).
__device__ __forceinline__ void copy_elem(void* dst, int64_t dst_i, int dst_dtype, const void* src, int64_t src_i,
                                          int src_dtype) {
  if (dst_dtype == src_dtype) {
    if (dst_dtype == 2)
      reinterpret_cast<uint32_t*>(dst)[dst_i] = reinterpret_cast<const uint32_t*>(src)[src_i];
    else
      reinterpret_cast<uint16_t*>(dst)[dst_i] = reinterpret_cast<const uint16_t*>(src)[src_i];
    return;
  }
  const float x = load_as_f32(src, src_i, src_dtype);
  if (dst_dtype == 2) {
    reinterpret_cast<float*>(dst)[dst_i] = x;
  } else if (dst_dtype == 1) {
    reinterpret_cast<_Float16*>(dst)[dst_i] = (_Float16)x;
  } else {
    reinterpret_cast<uint16_t*>(dst)[dst_i] = (uint16_t)(ElemBF16::pack2(x, 0.f) & 0xffffu);
  }
}

}  // namespace

// Fast path (same dtype, 16-byte aligned rows, H <= kMaxVecHeads): the old lengths go to LDS and
// every 16-byte piece of the four new rows is loaded at the same time, so the update costs one load
// round trip; after one barrier the pieces are stored and the lengths advanced (every reader takes
// the old lengths from LDS, so the new values can be written at once). Pieces are numbered (row r
// in {ring K, ring V, retained K, retained V}, head, piece).
constexpr int kPieceBatch = 4;

__global__ __launch_bounds__(256) void kv_update_vec_kernel(const KvUpdateArgs a) {
  __shared__ int64_t s_len[kMaxVecHeads];
  __shared__ int64_t s_ring[2];
  const int b = blockIdx.x, tid = threadIdx.x;
  // The active flag is loaded with everything else (an inactive sequence's loads are in bounds and
  // harmless) and tested once those are in flight, before anything is stored.
  const bool act = cache_flag_load(a.active, (int64_t)b * a.active_sb, a.active_bytes);
  const bool ring = a.window > 0;
  for (int h = tid; h < a.H; h += 256) s_len[h] = cache_len_load(a.ret_len, b * a.ret_len_sb + h * a.ret_len_sh, a.len_i64);
  if (ring && tid == 0) {
    s_ring[0] = cache_len_load(a.ring_len, (int64_t)b * a.ring_len_sb, a.len_i64);
    s_ring[1] = cache_len_load(a.ring_pos, (int64_t)b * a.ring_pos_sb, a.len_i64);
  }
  const int esz = a.kv_dtype == 2 ? 4 : 2;
  const int ppr = a.D * esz / 16;  // 16-byte pieces per row
  const int per_row_set = a.H * ppr;
  const int first_row = ring ? 0 : 2;
  const int total = (4 - first_row) * per_row_set;
  for (int base = 0; base < total; base += 256 * kPieceBatch) {
    uint4 val[kPieceBatch];
#pragma unroll
    for (int u = 0; u < kPieceBatch; ++u) {
      const int c = base + u * 256 + tid;
      if (c < total) {
        const int r = first_row + c / per_row_set, rem = c % per_row_set, h = rem / ppr, j = rem - h * ppr;
        const void* src = r == 0 ? a.kw : r == 1 ? a.vw : r == 2 ? a.kr : a.vr;
        const int64_t sb = r == 0 ? a.kw_sb : r == 1 ? a.vw_sb : r == 2 ? a.kr_sb : a.vr_sb;
        const int64_t sh = r == 0 ? a.kw_sh : r == 1 ? a.vw_sh : r == 2 ? a.kr_sh : a.vr_sh;
        val[u] = *reinterpret_cast<const uint4*>(static_cast<const char*>(src) + (b * sb + h * sh) * esz + j * 16);
      }
    }
    if (base == 0) {
      if (!act) return;  // whole workgroup
      __syncthreads();   // old lengths in LDS (uniform: every thread takes the first batch)
    }
    const int64_t rlen = ring ? s_ring[0] : 0, rpos = ring ? s_ring[1] : 0;
    const int64_t slot = rlen >= a.window ? rpos : rlen;
    const bool ring_write = ring && slot >= 0 && slot < a.ring_storage;
#pragma unroll
    for (int u = 0; u < kPieceBatch; ++u) {
      const int c = base + u * 256 + tid;
      if (c >= total) continue;
      const int r = first_row + c / per_row_set, rem = c % per_row_set, h = rem / ppr, j = rem - h * ppr;
      int64_t t;
      if (r < 2) {
        if (!ring_write) continue;
        t = slot;
      } else {
        t = s_len[h];
        if (t < 0 || t >= a.ret_storage) continue;
      }
      void* dst = r == 0 ? a.ring_k : r == 1 ? a.ring_v : r == 2 ? a.ret_k : a.ret_v;
      const int64_t db = r == 0 ? a.rk_sb : r == 1 ? a.rv_sb : r == 2 ? a.tk_sb : a.tv_sb;
      const int64_t dh = r == 0 ? a.rk_sh : r == 1 ? a.rv_sh : r == 2 ? a.tk_sh : a.tv_sh;
      const int64_t dt = r == 0 ? a.rk_st : r == 1 ? a.rv_st : r == 2 ? a.tk_st : a.tv_st;
      *reinterpret_cast<uint4*>(static_cast<char*>(dst) + (b * db + h * dh + t * dt) * esz + j * 16) = val[u];
    }
  }
  if (ring && tid == 0) {
    if (s_ring[0] >= a.window)
      cache_len_store(a.ring_pos, (int64_t)b * a.ring_pos_sb, a.len_i64, (s_ring[1] + 1) % a.window);
    else
      cache_len_store(a.ring_len, (int64_t)b * a.ring_len_sb, a.len_i64, s_ring[0] + 1);
  }
  for (int h = tid; h < a.H; h += 256) {
    const int64_t n = s_len[h];
    if (n >= 0 && n < a.ret_storage) cache_len_store(a.ret_len, b * a.ret_len_sb + h * a.ret_len_sh, a.len_i64, n + 1);
  }
}

// General path (dtype conversion or rows not 16-byte aligned): element by element.
__global__ __launch_bounds__(256) void kv_update_kernel(const KvUpdateArgs a) {
  const int b = blockIdx.x, tid = threadIdx.x;
  if (!cache_flag_load(a.active, (int64_t)b * a.active_sb, a.active_bytes)) return;  // whole workgroup
  const bool ring = a.window > 0;
  int64_t rlen = 0, rpos = 0;
  if (ring) {
    rlen = cache_len_load(a.ring_len, (int64_t)b * a.ring_len_sb, a.len_i64);
    rpos = cache_len_load(a.ring_pos, (int64_t)b * a.ring_pos_sb, a.len_i64);
  }
  const bool full = rlen >= a.window;
  const int64_t slot = full ? rpos : rlen;
  const bool ring_write = ring && slot >= 0 && slot < a.ring_storage;
  const int HD = a.H * a.D;
  for (int idx = tid; idx < HD; idx += 256) {
    const int h = idx / a.D, d = idx - h * a.D;
    if (ring_write) {
      copy_elem(a.ring_k, b * a.rk_sb + h * a.rk_sh + slot * a.rk_st + d, a.kv_dtype, a.kw,
                b * a.kw_sb + h * a.kw_sh + d, a.new_dtype);
      copy_elem(a.ring_v, b * a.rv_sb + h * a.rv_sh + slot * a.rv_st + d, a.kv_dtype, a.vw,
                b * a.vw_sb + h * a.vw_sh + d, a.new_dtype);
    }
    const int64_t len = cache_len_load(a.ret_len, b * a.ret_len_sb + h * a.ret_len_sh, a.len_i64);
    if (len >= 0 && len < a.ret_storage) {
      copy_elem(a.ret_k, b * a.tk_sb + h * a.tk_sh + len * a.tk_st + d, a.kv_dtype, a.kr,
                b * a.kr_sb + h * a.kr_sh + d, a.new_dtype);
      copy_elem(a.ret_v, b * a.tv_sb + h * a.tv_sh + len * a.tv_st + d, a.kv_dtype, a.vr,
                b * a.vr_sb + h * a.vr_sh + d, a.new_dtype);
    }
  }
  __syncthreads();  // every thread has read the old lengths before any is advanced
  if (ring && tid == 0) {
    if (full)
      cache_len_store(a.ring_pos, (int64_t)b * a.ring_pos_sb, a.len_i64, (rpos + 1) % a.window);
    else
      cache_len_store(a.ring_len, (int64_t)b * a.ring_len_sb, a.len_i64, rlen + 1);
  }
  for (int h = tid; h < a.H; h += 256) {
    const int64_t off = b * a.ret_len_sb + h * a.ret_len_sh;
    const int64_t len = cache_len_load(a.ret_len, off, a.len_i64);
    if (len >= 0 && len < a.ret_storage) cache_len_store(a.ret_len, off, a.len_i64, len + 1);
  }
}

hipError_t launch_kv_update(const KvUpdateArgs& a, hipStream_t stream) {
  if (a.B == 0 || a.H == 0 || a.D == 0) return hipSuccess;
  if (a.vec16)
    hipLaunchKernelGGL(kv_update_vec_kernel, dim3(a.B), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL(kv_update_kernel, dim3(a.B), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace sps
