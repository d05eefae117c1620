// Pre-attention fusion: rotary position embedding of Q and K plus the cast of Q, K, V to the
// attention dtype, in one pass over the projections, written in [B, N, H, D] memory order (the
// attention entry points take the [B, H, N, D] transposed views of these buffers as they are).
//
// Reference: apply_rotary_emb (model.py:201-230) followed by the transposes and casts of the
// attention callers (sps/core.py:45-55, reverse_sps/core.py:60-75): each (re, im) pair of a head
// row, (x[2i], x[2i+1]), is multiplied in fp32 by the position's complex frequency freqs_cis[n, i]
// (or freqs_cis[b, n, i] for per-sequence positions, model.py:160-199):
//   out[2i] = x[2i] * f.re - x[2i+1] * f.im,   out[2i+1] = x[2i] * f.im + x[2i+1] * f.re,
// then rounded once to the output dtype (round to nearest even). V is only cast.
//
// HBM-bound: one thread per 8-element piece of a (b, n, h) row of each of Q, K, V.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "cdna4.hpp"
#include "decode_kernels.hpp"

namespace sps {


namespace {

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

}  // namespace

__global__ __launch_bounds__(256) void rope_qkv_kernel(const RopeArgs a) {
  const int pieces = a.D / 8;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = (int64_t)a.B * a.N * a.H * pieces;
  if (idx >= total) return;
  const int c = (int)(idx % pieces);
  int64_t r = idx / pieces;
  const int h = (int)(r % a.H);
  r /= a.H;
  const int n = (int)(r % a.N);
  const int b = (int)(r / a.N);
  const int d0 = 8 * c;

  // This piece's four complex frequencies (pairs d0/2 .. d0/2 + 3).
  const float* fr = a.freqs + b * a.f_sb + n * a.f_sn + d0;
  const f32x4_t f01 = *reinterpret_cast<const f32x4_t*>(fr);
  const f32x4_t f23 = *reinterpret_cast<const f32x4_t*>(fr + 4);
  const float fre[4] = {f01[0], f01[2], f23[0], f23[2]};
  const float fim[4] = {f01[1], f01[3], f23[1], f23[3]};

  float x[8], y[8];
  load8(a.q, b * a.q_sb + n * a.q_sn + h * a.q_sh + d0, a.in_dtype, x);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    y[2 * i] = x[2 * i] * fre[i] - x[2 * i + 1] * fim[i];
    y[2 * i + 1] = x[2 * i] * fim[i] + x[2 * i + 1] * fre[i];
  }
  store8(a.qo, b * a.qo_sb + n * a.qo_sn + h * a.qo_sh + d0, a.out_dtype, y);
  load8(a.k, b * a.k_sb + n * a.k_sn + h * a.k_sh + d0, a.in_dtype, x);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    y[2 * i] = x[2 * i] * fre[i] - x[2 * i + 1] * fim[i];
    y[2 * i + 1] = x[2 * i] * fim[i] + x[2 * i + 1] * fre[i];
  }
  store8(a.ko, b * a.ko_sb + n * a.ko_sn + h * a.ko_sh + d0, a.out_dtype, y);
  if (a.v) {
    load8(a.v, b * a.v_sb + n * a.v_sn + h * a.v_sh + d0, a.in_dtype, x);
    store8(a.vo, b * a.vo_sb + n * a.vo_sn + h * a.vo_sh + d0, a.out_dtype, x);
  }
}

hipError_t launch_rope_qkv(const RopeArgs& a, hipStream_t stream) {
  const int64_t total = (int64_t)a.B * a.N * a.H * (a.D / 8);
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(rope_qkv_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace sps
