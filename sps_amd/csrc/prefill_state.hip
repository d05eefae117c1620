// Prefill -> decode state: after a prompt's batched prefill, the current document's K/V rows of one
// layer go into the decode caches (retained buffer: every token of the document; ring: its last
// window_tokens tokens), one launch for the whole batch instead of a per-row host loop.
//
// Reference: _materialize_prefill_layer_state (reverse_sps/inference.py:568-613). Per sequence b,
// doc = the token positions t with current_doc_mask[b, t] set, in increasing order (n = |doc|;
// rows with n == 0 are left untouched):
//   retained K/V[b, :, j, :] = K/V[b, 2 doc[j] + retained_slot, :, :]  (j < n), ret_len[b, :] = n
//   ring (window_tokens > 0): w = min(n, window_tokens), ring K/V[b, :, i, :] =
//     K/V[b, 2 doc[n - w + i] + window_slot, :, :] (i < w), ring_len[b] = w, ring_pos[b] = 0,
// with the rows converted to the cache dtype (round to nearest even).
//
// kPfSplit workgroups per (head, sequence): each compacts the mask row into an LDS list of positions
// in chunks (a shuffle scan gives each set position its rank; the row is a few KB, read from L2 by
// every split), then copies every kPfSplit-th group of rows with groups of D/8 threads moving
// 16-byte pieces, so a long document is copied by many workgroups at once.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "cdna4.hpp"
#include "decode_kernels.hpp"

namespace sps {

namespace {

constexpr int kPfThreads = 256;
constexpr int kPfChunk = 2048;  // positions compacted per pass
constexpr int kPfSplit = 8;     // workgroups per (head, sequence)

__device__ __forceinline__ void load8(const void* p, int64_t i, int dtype, float* x) {
  if (dtype == 2) {
    const f32x4_t a = *reinterpret_cast<const f32x4_t*>(static_cast<const float*>(p) + i);
    const f32x4_t b = *reinterpret_cast<const f32x4_t*>(static_cast<const float*>(p) + i + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = a[e];
      x[4 + e] = b[e];
    }
  } else {
    const u32x4_t w = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(p) + i);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t u = w[e];
      x[2 * e] = dtype == 1 ? ElemF16::to_f32((uint16_t)(u & 0xffffu)) : ElemBF16::to_f32((uint16_t)(u & 0xffffu));
      x[2 * e + 1] = dtype == 1 ? ElemF16::to_f32((uint16_t)(u >> 16)) : ElemBF16::to_f32((uint16_t)(u >> 16));
    }
  }
}

__device__ __forceinline__ void store8(void* p, int64_t i, int dtype, const float* x) {
  if (dtype == 2) {
    f32x4_t a, b;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      a[e] = x[e];
      b[e] = x[4 + e];
    }
    *reinterpret_cast<f32x4_t*>(static_cast<float*>(p) + i) = a;
    *reinterpret_cast<f32x4_t*>(static_cast<float*>(p) + i + 4) = b;
  } else {
    u32x4_t w;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w[e] = dtype == 1 ? ElemF16::pack2(x[2 * e], x[2 * e + 1]) : ElemBF16::pack2(x[2 * e], x[2 * e + 1]);
    *reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(p) + i) = w;
  }
}

// Exclusive prefix sum over the workgroup's threads (shuffle scan per wave, wave totals in LDS).
__device__ int block_exclusive_sum(int x, int* s_tot, int& total) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int v = x;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(v, o);
    if (lane >= o) v += y;
  }
  if (lane == 63) s_tot[wave] = v;
  __syncthreads();
  int carry = 0;
  total = 0;
#pragma unroll
  for (int w = 0; w < kPfThreads / 64; ++w) {
    const int t = s_tot[w];
    carry += w < wave ? t : 0;
    total += t;
  }
  __syncthreads();
  return carry + v - x;
}

}  // namespace

__global__ __launch_bounds__(kPfThreads) void prefill_state_kernel(const PrefillStateArgs a) {
  __shared__ int s_pos[kPfChunk];
  __shared__ int s_tot[kPfThreads / 64];
  const int h = blockIdx.x, b = blockIdx.y, split = blockIdx.z, tid = threadIdx.x;
  const uint8_t* mrow = a.mask + (int64_t)b * a.mask_sb;

  // Pass 1: the document's length.
  int cnt = 0;
  for (int t = tid; t < a.T; t += kPfThreads) cnt += mrow[t] != 0;
  int n;
  block_exclusive_sum(cnt, s_tot, n);
  if (n == 0) return;  // untouched, as in the reference (uniform over the workgroup)
  const int w = a.window > 0 ? (n < a.window ? n : a.window) : 0;
  const int first_w = n - w;

  // Pass 2: compact the set positions chunk by chunk (rank order) and copy their rows.
  const int pieces = a.D / 8;
  const int rows_per_pass = kPfThreads / pieces;
  const int r_in = tid / pieces, piece = tid - r_in * pieces;
  int base = 0;  // ranks before this chunk
  for (int c0 = 0; c0 < a.T; c0 += kPfChunk) {
    const int span = (a.T - c0) < kPfChunk ? (a.T - c0) : kPfChunk;
    const int per = (span + kPfThreads - 1) / kPfThreads;  // contiguous positions per thread
    const int p0 = c0 + tid * per, p1 = p0 + per < c0 + span ? p0 + per : c0 + span;
    int mine = 0;
    for (int t = p0; t < p1; ++t) mine += mrow[t] != 0;
    int chunk_total;
    int rank = block_exclusive_sum(mine, s_tot, chunk_total);
    for (int t = p0; t < p1; ++t)
      if (mrow[t] != 0) s_pos[rank++] = t;
    __syncthreads();
    if (r_in < rows_per_pass) {
      for (int r = r_in + split * rows_per_pass; r < chunk_total; r += rows_per_pass * kPfSplit) {
        const int j = base + r;  // rank of this position in the document
        const int t = s_pos[r];
        float x[8];
        if (j < a.ret_storage) {
          load8(a.k, b * a.k_sb + (int64_t)(2 * t + a.retained_slot) * a.k_sn + h * a.k_sh + 8 * piece, a.in_dtype, x);
          store8(a.ret_k, b * a.tk_sb + h * a.tk_sh + (int64_t)j * a.tk_st + 8 * piece, a.kv_dtype, x);
          load8(a.v, b * a.v_sb + (int64_t)(2 * t + a.retained_slot) * a.v_sn + h * a.v_sh + 8 * piece, a.in_dtype, x);
          store8(a.ret_v, b * a.tv_sb + h * a.tv_sh + (int64_t)j * a.tv_st + 8 * piece, a.kv_dtype, x);
        }
        const int i = j - first_w;
        if (a.window > 0 && i >= 0 && i < a.ring_storage) {
          load8(a.k, b * a.k_sb + (int64_t)(2 * t + a.window_slot) * a.k_sn + h * a.k_sh + 8 * piece, a.in_dtype, x);
          store8(a.ring_k, b * a.rk_sb + h * a.rk_sh + (int64_t)i * a.rk_st + 8 * piece, a.kv_dtype, x);
          load8(a.v, b * a.v_sb + (int64_t)(2 * t + a.window_slot) * a.v_sn + h * a.v_sh + 8 * piece, a.in_dtype, x);
          store8(a.ring_v, b * a.rv_sb + h * a.rv_sh + (int64_t)i * a.rv_st + 8 * piece, a.kv_dtype, x);
        }
      }
    }
    base += chunk_total;
    __syncthreads();  // s_pos is rewritten by the next chunk
  }
  if (tid == 0 && split == 0) {
    const int64_t nl = n < a.ret_storage ? n : a.ret_storage;
    const int64_t off = b * a.ret_len_sb + h * a.ret_len_sh;
    if (a.len_i64) reinterpret_cast<int64_t*>(a.ret_len)[off] = nl;
    else reinterpret_cast<int*>(a.ret_len)[off] = (int)nl;
    if (a.window > 0 && h == 0) {
      if (a.len_i64) {
        reinterpret_cast<int64_t*>(a.ring_len)[b * a.ring_len_sb] = w;
        reinterpret_cast<int64_t*>(a.ring_pos)[b * a.ring_pos_sb] = 0;
      } else {
        reinterpret_cast<int*>(a.ring_len)[b * a.ring_len_sb] = w;
        reinterpret_cast<int*>(a.ring_pos)[b * a.ring_pos_sb] = 0;
      }
    }
  }
}

hipError_t launch_prefill_state(const PrefillStateArgs& a, hipStream_t stream) {
  if (a.B == 0 || a.H == 0 || a.T == 0) return hipSuccess;
  hipLaunchKernelGGL(prefill_state_kernel, dim3(a.H, a.B, kPfSplit), dim3(kPfThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace sps
