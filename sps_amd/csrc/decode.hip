// Segmented decode attention (1 or 2 queries per (batch, head)) over up to 3 variable-length KV
// segments plus up to 2 single-token "extra" keys, gfx950.
//
// Reference semantics: _segmented_q1_attention_kernel / _segmented_q2_attention_kernel
// (utils/decode_attention.py:79-188, 267-368): fp32 scores from 16-bit K/V, online softmax,
// key t of a segment is valid iff t < min(max(len, 0), scan_len), output 0 when no key is valid.
// Extras are always valid; in the q=2 form the first extra (current input key) is seen by both
// queries and the second (current <predict> key) by query 1 only.
//
// The pass is HBM-bound (one query row per 256 B of K+V at D = 64), so it is organised for
// bandwidth, not MFMA: every segment is cut into fixed chunks of keys, one workgroup per
// (chunk, head, batch). Each wave streams its slice of the chunk with 16-byte coalesced loads
// (all loads issued before any arithmetic; nontemporal, since every K/V byte is read once: at
// the benchmark shape this alone takes the kernel from 5.6 to 6.2 TB/s and leaves L2 to the
// partial records the merge reads), computes fp32 dot products with a short lane
// reduction, and keeps an exp2-domain partial softmax; the four waves merge in LDS and the
// workgroup writes one (acc[D], m, l) partial. Only live keys are read: chunks past the live
// length exit before touching K/V. A second small kernel merges the partials with the extras: one
// wave per (sequence, head, query slot), lanes over chunks for the max and the sums, then batched
// coalesced reads of the accumulators (no chain of dependent loads per chunk).
//
// KV update in the same launch (sps_decode_kv_update; reference decode step: the attention over the
// caches, then fused_sps_kv_update, reverse_sps/inference.py:169-238, 437-470). The update writes the
// rows and lengths the attention reads, so the two must not overlap: the partial kernel reads every
// cache row before the merge kernel starts (stream order), and the first-chunk workgroup of each
// (sequence, head), which the grid always launches, stores the old lengths in a snapshot. The merge
// kernel reads only the snapshot: its query-0 wave of each (sequence, head) writes that head's new
// ring and retained rows and advances its retained length; the wave of head 0 advances the ring's
// length or position. No wave of the launch reads a length another one writes.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "cdna4.hpp"
#include "decode_kernels.hpp"

namespace sps {

struct KvBF16 {
  using raw = uint16_t;
  static __device__ __forceinline__ float cvt(uint16_t x) { return ElemBF16::to_f32(x); }
};
struct KvF16 {
  using raw = uint16_t;
  static __device__ __forceinline__ float cvt(uint16_t x) { return ElemF16::to_f32(x); }
};
struct KvF32 {
  using raw = float;
  static __device__ __forceinline__ float cvt(float x) { return x; }
};

template <class KV>
__device__ __forceinline__ void unpack16(const u32x4_t w, float* out) {
  if constexpr (sizeof(typename KV::raw) == 2) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = KV::cvt((uint16_t)(w[i] & 0xffffu));
      out[2 * i + 1] = KV::cvt((uint16_t)(w[i] >> 16));
    }
  } else {
    // Copy each element to a scalar first: clang lowers __builtin_bit_cast of a vector-element
    // subscript (an lvalue) as a read of element 0.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t x = w[i];
      out[i] = __builtin_bit_cast(float, x);
    }
  }
}

__device__ __forceinline__ int imin_d(int x, int y) { return x < y ? x : y; }

__device__ __forceinline__ int seg_live_len(const DecodeSeg& sg, int b, int h, int H) {
  if (sg.scan == 0) return 0;
  const int64_t idx = sg.len_per_head ? (int64_t)b * H + h : b;
  int64_t len = sg.len_i64 ? reinterpret_cast<const int64_t*>(sg.len)[idx]
                           : (int64_t) reinterpret_cast<const int32_t*>(sg.len)[idx];
  if (len < 0) len = 0;
  if (len > sg.scan) len = sg.scan;
  return (int)len;
}

// Sum over aligned groups of W lanes (W <= 16 by DPP moves inside each 16-lane row: quad swaps,
// then the half-row and row mirrors; every lane of the group receives the sum). Larger groups finish
// with cross-row shuffles.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

template <int W>
__device__ __forceinline__ float row_group_sum(float x) {
  if constexpr (W >= 2) x += dpp_f<0xB1>(x);    // quad_perm [1, 0, 3, 2]
  if constexpr (W >= 4) x += dpp_f<0x4E>(x);    // quad_perm [2, 3, 0, 1]
  if constexpr (W >= 8) x += dpp_f<0x141>(x);   // row_half_mirror
  if constexpr (W >= 16) x += dpp_f<0x140>(x);  // row_mirror
#pragma unroll
  for (int o = 16; o < W; o <<= 1) x += __shfl_xor(x, o);
  return x;
}

template <int W>
__device__ __forceinline__ float xor_sum(float x) {
#pragma unroll
  for (int o = 1; o < W; o <<= 1) x += __shfl_xor(x, o);
  return x;
}

// Reduction over lanes that differ only in bits [log2(LPR), 6): the row groups of a wave.
template <int LPR>
__device__ __forceinline__ float group_max(float x) {
#pragma unroll
  for (int o = LPR; o < 64; o <<= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}
template <int LPR>
__device__ __forceinline__ float group_sum(float x) {
#pragma unroll
  for (int o = LPR; o < 64; o <<= 1) x += __shfl_xor(x, o);
  return x;
}

// Packed dot product of 8 16-bit elements (v_dot2_f32_bf16 / v_dot2_f32_f16: exact products,
// fp32 accumulation) for K/V and query in the same 16-bit type.
template <class KV>
__device__ __forceinline__ float dot8_packed(u32x4_t k, u32x4_t q, float acc) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    // Elements copied to scalars first: clang lowers __builtin_bit_cast of a vector-element
    // subscript (an lvalue) as a read of element 0.
    const uint32_t ki = k[i], qi = q[i];
    if constexpr (std::is_same<KV, KvBF16>::value)
      acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, ki), __builtin_bit_cast(bf16x2_t, qi), acc,
                                           false);
    else
      acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, ki), __builtin_bit_cast(f16x2_t, qi), acc, false);
  }
  return acc;
}

// The lengths the merge kernel and the folded KV update use, as they are before the update (one
// thread of the (b, h)'s first-chunk workgroup).
__device__ __forceinline__ void snapshot_lengths(const DecodeArgs& a, int b, int h) {
  int64_t* sn = a.snap + ((int64_t)b * a.H + h) * kSnapWords;
  for (int s = 0; s < a.n_seg; ++s) sn[s] = seg_live_len(a.seg[s], b, h, a.H);
  const KvUpdateArgs& u = a.upd;
  sn[kSnapRingLen] = u.window > 0 ? cache_len_load(u.ring_len, (int64_t)b * u.ring_len_sb, u.len_i64) : 0;
  sn[kSnapRingPos] = u.window > 0 ? cache_len_load(u.ring_pos, (int64_t)b * u.ring_pos_sb, u.len_i64) : 0;
  sn[kSnapRetLen] = cache_len_load(u.ret_len, b * u.ret_len_sb + h * u.ret_len_sh, u.len_i64);
  sn[kSnapActive] = cache_flag_load(u.active, (int64_t)b * u.active_sb, u.active_bytes);
}

// PQ: the query is in the K/V's 16-bit type with 16-byte aligned rows (the host checks), so the
// scores are packed dot products of raw K words and raw query words, with no conversion of K.
// Three waves per SIMD: the two-query form otherwise compiles to 170 VGPRs, one wave per SIMD fewer
// than at 168, which measured 6 % slower at C5 (q = 2: 117.3 against 110.5 us); at D = 16 the
// 168-register budget would spill 18 VGPRs, so that head dim keeps the compiler's choice.
template <int D, int NQ, class KV, bool PQ>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D == 16 ? 1 : 3, 8))) void decode_partial_kernel(
    const DecodeArgs a) {
  constexpr int EPL = 16 / (int)sizeof(typename KV::raw);  // elements per 16-byte load
  constexpr int LPR = D / EPL;                              // lanes per key row
  constexpr int RPP = 64 / LPR;                             // rows per wave pass
  constexpr int PASS = DecodeGeom<D, sizeof(typename KV::raw)>::PASS;
  constexpr int KW = RPP * PASS;                            // keys per wave
  constexpr int CK = 4 * KW;                                // keys per workgroup chunk
  static_assert(CK == DecodeGeom<D, sizeof(typename KV::raw)>::CHUNK, "chunk geometry");
  __shared__ float s_m[4][NQ], s_l[4][NQ];
  __shared__ __attribute__((aligned(16))) float s_acc[4][NQ][D];

  const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  if (a.snap && c == 0 && threadIdx.x == 0) snapshot_lengths(a, b, h);
  int si = 0;
  while (si + 1 < a.n_seg && c >= a.seg[si + 1].chunk_base) ++si;
  const DecodeSeg sg = a.seg[si];
  const int live = seg_live_len(sg, b, h, a.H);
  const int t0 = (c - sg.chunk_base) * CK;
  if (t0 >= live) return;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane / LPR, cc = lane % LPR;

  // This lane's query slice(s): elements cc*EPL .. +EPL (fp32, or raw 16-bit words when PQ).
  float qv[NQ][PQ ? 1 : EPL];
  u32x4_t qw[NQ];
#pragma unroll
  for (int qi = 0; qi < NQ; ++qi) {
    const int64_t q0 = b * a.q_sb + qi * a.q_ss + h * a.q_sh + cc * EPL;
    if constexpr (PQ) {
      qw[qi] = *reinterpret_cast<const u32x4_t*>(reinterpret_cast<const uint16_t*>(a.q) + q0);
    } else {
#pragma unroll
      for (int e = 0; e < EPL; ++e) qv[qi][e] = load_as_f32(a.q, q0 + e, a.q_dtype);
    }
  }

  using raw_t = typename KV::raw;
  const raw_t* kb = reinterpret_cast<const raw_t*>(sg.k) + b * sg.ksb + h * sg.ksh + cc * EPL;
  const raw_t* vb = reinterpret_cast<const raw_t*>(sg.v) + b * sg.vsb + h * sg.vsh + cc * EPL;
  const int tw = t0 + wave * KW + r;
  u32x4_t kr[PASS], vr[PASS];
#pragma unroll
  for (int j = 0; j < PASS; ++j) {
    const int t = tw + j * RPP;
    u32x4_t z = {0u, 0u, 0u, 0u};
    kr[j] = t < live ? __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(kb + (int64_t)t * sg.kst)) : z;
  }
#pragma unroll
  for (int j = 0; j < PASS; ++j) {
    const int t = tw + j * RPP;
    u32x4_t z = {0u, 0u, 0u, 0u};
    vr[j] = t < live ? __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(vb + (int64_t)t * sg.vst)) : z;
  }

  float sc[NQ][PASS];
#pragma unroll
  for (int j = 0; j < PASS; ++j) {
    float kf[PQ ? 1 : EPL];
    if constexpr (!PQ) unpack16<KV>(kr[j], kf);
#pragma unroll
    for (int qi = 0; qi < NQ; ++qi) {
      float d = 0.f;
      if constexpr (PQ) {
        d = dot8_packed<KV>(kr[j], qw[qi], d);
      } else {
#pragma unroll
        for (int e = 0; e < EPL; ++e) d = fmaf(qv[qi][e], kf[e], d);
      }
      d = row_group_sum<LPR>(d);
      sc[qi][j] = (tw + j * RPP < live) ? d * a.scale2 : -INFINITY;
    }
  }

  float acc[NQ][EPL];
  float mw[NQ], lw[NQ];
#pragma unroll
  for (int qi = 0; qi < NQ; ++qi) {
    float mx = sc[qi][0];
#pragma unroll
    for (int j = 1; j < PASS; ++j) mx = fmaxf(mx, sc[qi][j]);
    mx = group_max<LPR>(mx);
    const float mu = mx == -INFINITY ? 0.f : mx;
    float l = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[qi][e] = 0.f;
#pragma unroll
    for (int j = 0; j < PASS; ++j) {
      const float p = fast_exp2(sc[qi][j] - mu);
      l += p;
      float vf[EPL];
      unpack16<KV>(vr[j], vf);
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[qi][e] = fmaf(p, vf[e], acc[qi][e]);
    }
    mw[qi] = mx;
    lw[qi] = group_sum<LPR>(l);
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[qi][e] = group_sum<LPR>(acc[qi][e]);
  }

  if (r == 0) {
#pragma unroll
    for (int qi = 0; qi < NQ; ++qi) {
#pragma unroll
      for (int e = 0; e < EPL; ++e) s_acc[wave][qi][cc * EPL + e] = acc[qi][e];
      if (cc == 0) {
        s_m[wave][qi] = mw[qi];
        s_l[wave][qi] = lw[qi];
      }
    }
  }
  __syncthreads();
  constexpr int REC = DecodeGeom<D, 2>::REC;
  float* out = a.part + (((int64_t)(b * a.H + h) * a.n_chunks + c) * NQ) * REC;
  for (int i = tid; i < NQ * D; i += 256) {
    const int qi = i / D, d = i - qi * D;
    float M = s_m[0][qi];
#pragma unroll
    for (int w = 1; w < 4; ++w) M = fmaxf(M, s_m[w][qi]);
    const float mu = M == -INFINITY ? 0.f : M;
    float A = 0.f, L = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float f = fast_exp2(s_m[w][qi] - mu);
      A = fmaf(f, s_acc[w][qi][d], A);
      L = fmaf(f, s_l[w][qi], L);
    }
    out[qi * REC + d] = A;
    if (d == 0) {
      out[qi * REC + D] = M;
      out[qi * REC + D + 1] = L;
    }
  }
}

// Index of the k-th live chunk of (b, h) over the segments in order (chunks of segment s are
// chunk_base[s] .. chunk_base[s] + nc[s] - 1).
__device__ __forceinline__ int live_chunk(const DecodeArgs& a, const int* nc, int k) {
  for (int s = 0; s < a.n_seg; ++s) {
    if (k < nc[s]) return a.seg[s].chunk_base + k;
    k -= nc[s];
  }
  return -1;
}

template <int N>
__device__ __forceinline__ float wave_max_f(float x) {
#pragma unroll
  for (int o = 1; o < N; o <<= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}

// One wave per (query slot, head, batch): merges the chunk partials and the extra keys, normalises
// and writes fp32. Everything that depends only on the chunk list is loaded in one round trip
// before the max reduction: the extra keys' rows, each lane's chunk maximum and weight sum (lanes own
// chunks, in rounds of 64), and the accumulator rows of the first kMergeAhead chunks (lanes over d).
// Chunks beyond those are read 8 records per batch after the max is known.
constexpr int kMergeAhead = 16;

template <int D, int NQ>
__global__ __launch_bounds__(64) void decode_merge_kernel(const DecodeArgs a) {
  constexpr int DPL = (D + 63) / 64;  // output elements per lane
  constexpr int REC = DecodeGeom<D, 2>::REC;
  const int qi = blockIdx.x, h = blockIdx.y, b = blockIdx.z, lane = threadIdx.x;
  // With the KV update folded in, lengths come from the snapshot only (this launch writes them).
  const int64_t* snap = a.snap ? a.snap + ((int64_t)b * a.H + h) * kSnapWords : nullptr;
  const bool upd = snap && qi == 0;
  // The update's new rows, 16-byte pieces numbered (row r in {ring K, ring V, retained K, retained
  // V}, piece j), loaded first: nothing else depends on them, and they are stored at the end.
  constexpr int kUpdPieces = 4;  // per lane: 4 rows of at most 1 KiB (D = 256 in fp32)
  u32x4_t uval[kUpdPieces];
  int upr = 0;
  if (upd) {
    const KvUpdateArgs& u = a.upd;
    upr = u.D * (u.kv_dtype == 2 ? 4 : 2) / 16;
#pragma unroll
    for (int i = 0; i < kUpdPieces; ++i) {
      const int pc = lane + 64 * i, r = pc / upr, j = pc - r * upr;
      if (r < 4 && (r >= 2 || u.window > 0)) {
        const void* src = r == 0 ? u.kw : r == 1 ? u.vw : r == 2 ? u.kr : u.vr;
        const int64_t sb = r == 0 ? u.kw_sb : r == 1 ? u.vw_sb : r == 2 ? u.kr_sb : u.vr_sb;
        const int64_t sh = r == 0 ? u.kw_sh : r == 1 ? u.vw_sh : r == 2 ? u.kr_sh : u.vr_sh;
        const int esz = u.kv_dtype == 2 ? 4 : 2;
        uval[i] = *reinterpret_cast<const u32x4_t*>(static_cast<const char*>(src) + (b * sb + h * sh) * esz + j * 16);
      }
    }
  }
  int nc[kMaxDecodeSegs] = {0, 0, 0};
  int total = 0;
  for (int s = 0; s < a.n_seg; ++s) {
    const int live = snap ? (int)snap[s] : seg_live_len(a.seg[s], b, h, a.H);
    nc[s] = (live + a.chunk_keys - 1) / a.chunk_keys;
    total += nc[s];
  }
  const float* part = a.part + ((int64_t)(b * a.H + h) * a.n_chunks) * NQ * REC + qi * REC;

  // The query slice and the extra keys' rows.
  const int64_t q0 = b * a.q_sb + qi * a.q_ss + h * a.q_sh;
  const int64_t e0 = b * a.e_sb + h * a.e_sh;
  float qd[DPL], ekd[kMaxDecodeExtras][DPL], evd[kMaxDecodeExtras][DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) {
    const int dd = lane + 64 * i;
    qd[i] = dd < D ? load_as_f32(a.q, q0 + dd, a.q_dtype) : 0.f;
  }
#pragma unroll
  for (int e = 0; e < kMaxDecodeExtras; ++e) {
#pragma unroll
    for (int i = 0; i < DPL; ++i) {
      const int dd = lane + 64 * i;
      const bool ld = e < a.n_extra && dd < D;
      ekd[e][i] = ld ? load_as_f32(a.ek[e], e0 + dd, a.e_dtype) : 0.f;
      evd[e][i] = ld ? load_as_f32(a.ev[e], e0 + dd, a.e_dtype) : 0.f;
    }
  }
  // This lane's chunk of the first round (chunk 0's record for idle lanes: in bounds).
  const int c0 = lane < total ? live_chunk(a, nc, lane) : -1;
  const float* r0 = part + (int64_t)(c0 < 0 ? 0 : c0) * NQ * REC;
  const float m0 = r0[D], l0 = r0[D + 1];
  // Accumulator rows of the first kMergeAhead chunks.
  float x[kMergeAhead][DPL];
#pragma unroll
  for (int u = 0; u < kMergeAhead; ++u) {
    const int cu = __shfl(c0, u);
    const float* ru = part + (int64_t)(cu < 0 ? 0 : cu) * NQ * REC;
#pragma unroll
    for (int i = 0; i < DPL; ++i) {
      const int dd = lane + 64 * i;
      x[u][i] = (u < total && dd < D) ? ru[dd] : 0.f;
    }
  }

  // Extra-key scores (all lanes hold them after the reduction).
  float es[kMaxDecodeExtras] = {-INFINITY, -INFINITY};
#pragma unroll
  for (int e = 0; e < kMaxDecodeExtras; ++e) {
    if (e >= a.n_extra) continue;
    float d = 0.f;
#pragma unroll
    for (int i = 0; i < DPL; ++i) d = fmaf(qd[i], ekd[e][i], d);
    d = xor_sum<64>(d);
    if ((a.emask[e] >> qi) & 1) es[e] = d * a.scale2;
  }

  // Max over chunk maxima and extra scores.
  float M = fmaxf(fmaxf(es[0], es[1]), c0 >= 0 ? m0 : -INFINITY);
  for (int k0 = 64; k0 < total; k0 += 64) {
    const int c = k0 + lane < total ? live_chunk(a, nc, k0 + lane) : -1;
    const float mc = part[(int64_t)(c < 0 ? 0 : c) * NQ * REC + D];  // in-bounds even for idle lanes
    M = fmaxf(M, c >= 0 ? mc : -INFINITY);
  }
  M = wave_max_f<64>(M);
  const float mu = M == -INFINITY ? 0.f : M;

  // Sum of weights and the weighted accumulators, chunk by chunk in order.
  float L = 0.f, A[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) A[i] = 0.f;
  // Accumulates the chunks [from, nk) of the round whose lane chunk / weight are (c, f).
  auto accumulate = [&](int c, float f, int from, int nk) {
    for (int j0 = from; j0 < nk; j0 += 8) {
      float fj[8];
      const float* rj[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int j = imin_d(j0 + u, nk - 1);
        fj[u] = j0 + u < nk ? __shfl(f, j) : 0.f;
        const int cj = __shfl(c, j);
        rj[u] = part + (int64_t)cj * NQ * REC;
      }
      float xr[8][DPL];
#pragma unroll
      for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int i = 0; i < DPL; ++i) {
          const int dd = lane + 64 * i;
          xr[u][i] = dd < D ? rj[u][dd] : 0.f;
        }
#pragma unroll
      for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int i = 0; i < DPL; ++i) A[i] = fmaf(fj[u], xr[u][i], A[i]);
    }
  };
  {
    const float f0 = c0 >= 0 ? fast_exp2(m0 - mu) : 0.f;
    L += c0 >= 0 ? f0 * l0 : 0.f;
    const int nk = imin_d(64, total);
#pragma unroll
    for (int u = 0; u < kMergeAhead; ++u) {
      const float fu = __shfl(f0, u);
      if (u < nk) {
#pragma unroll
        for (int i = 0; i < DPL; ++i) A[i] = fmaf(fu, x[u][i], A[i]);
      }
    }
    accumulate(c0, f0, kMergeAhead, nk);
  }
  for (int k0 = 64; k0 < total; k0 += 64) {
    const int c = k0 + lane < total ? live_chunk(a, nc, k0 + lane) : -1;
    const float* rec = part + (int64_t)(c < 0 ? 0 : c) * NQ * REC;
    const float mrec = rec[D], lrec = rec[D + 1];  // chunk 0's record for idle lanes: in bounds
    const float f = c >= 0 ? fast_exp2(mrec - mu) : 0.f;
    L += c >= 0 ? f * lrec : 0.f;
    accumulate(c, f, 0, imin_d(64, total - k0));
  }
  L = xor_sum<64>(L);
#pragma unroll
  for (int e = 0; e < kMaxDecodeExtras; ++e) {
    if (es[e] == -INFINITY) continue;
    const float f = fast_exp2(es[e] - mu);
    L += f;
#pragma unroll
    for (int i = 0; i < DPL; ++i) A[i] = fmaf(f, evd[e][i], A[i]);
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  float* orow = a.out + b * a.o_sb + qi * a.o_ss + h * a.o_sh;
#pragma unroll
  for (int i = 0; i < DPL; ++i) {
    const int dd = lane + 64 * i;
    if (dd < D) orow[dd] = A[i] * inv;
  }

  // The folded KV update of this (sequence, head), as sps_kv_update does it, from the old lengths.
  if (upd && snap[kSnapActive] != 0) {
    const KvUpdateArgs& u = a.upd;
    const int64_t rlen = snap[kSnapRingLen], rpos = snap[kSnapRingPos], tlen = snap[kSnapRetLen];
    const int64_t slot = rlen >= u.window ? rpos : rlen;
    const bool ring_write = u.window > 0 && slot >= 0 && slot < u.ring_storage;
    const bool ret_write = tlen >= 0 && tlen < u.ret_storage;
    const int esz = u.kv_dtype == 2 ? 4 : 2;
#pragma unroll
    for (int i = 0; i < kUpdPieces; ++i) {
      const int pc = lane + 64 * i, r = pc / upr, j = pc - r * upr;
      if (r >= 4 || !(r < 2 ? ring_write : ret_write)) continue;
      void* dst = r == 0 ? u.ring_k : r == 1 ? u.ring_v : r == 2 ? u.ret_k : u.ret_v;
      const int64_t db = r == 0 ? u.rk_sb : r == 1 ? u.rv_sb : r == 2 ? u.tk_sb : u.tv_sb;
      const int64_t dh = r == 0 ? u.rk_sh : r == 1 ? u.rv_sh : r == 2 ? u.tk_sh : u.tv_sh;
      const int64_t dt = r == 0 ? u.rk_st : r == 1 ? u.rv_st : r == 2 ? u.tk_st : u.tv_st;
      const int64_t t = r < 2 ? slot : tlen;
      *reinterpret_cast<u32x4_t*>(static_cast<char*>(dst) + (b * db + h * dh + t * dt) * esz + j * 16) = uval[i];
    }
    if (lane == 0) {
      if (ret_write) cache_len_store(u.ret_len, b * u.ret_len_sb + h * u.ret_len_sh, u.len_i64, tlen + 1);
      if (h == 0 && u.window > 0) {
        if (rlen >= u.window)
          cache_len_store(u.ring_pos, (int64_t)b * u.ring_pos_sb, u.len_i64, (rpos + 1) % u.window);
        else
          cache_len_store(u.ring_len, (int64_t)b * u.ring_len_sb, u.len_i64, rlen + 1);
      }
    }
  }
}

template <int D, int NQ, class KV>
static hipError_t launch_decode_t(const DecodeArgs& a, hipStream_t stream) {
  if (a.B == 0 || a.H == 0) return hipSuccess;
  if (a.n_chunks > 0) {
    constexpr bool k16 = sizeof(typename KV::raw) == 2;
    if (k16 && a.q_packed)
      hipLaunchKernelGGL((decode_partial_kernel<D, NQ, KV, k16>), dim3(a.n_chunks, a.H, a.B), dim3(256), 0,
                         stream, a);
    else
      hipLaunchKernelGGL((decode_partial_kernel<D, NQ, KV, false>), dim3(a.n_chunks, a.H, a.B), dim3(256), 0,
                         stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((decode_merge_kernel<D, NQ>), dim3(NQ, a.H, a.B), dim3(64), 0, stream, a);
  return hipGetLastError();
}

template <int D, int NQ>
static hipError_t launch_decode_kv(const DecodeArgs& a, int kv_dtype, hipStream_t stream) {
  switch (kv_dtype) {
    case 0:
      return launch_decode_t<D, NQ, KvBF16>(a, stream);
    case 1:
      return launch_decode_t<D, NQ, KvF16>(a, stream);
    case 2:
      return launch_decode_t<D, NQ, KvF32>(a, stream);
    default:
      return hipErrorInvalidValue;
  }
}

template <int D>
static hipError_t launch_decode_d(const DecodeArgs& a, int kv_dtype, hipStream_t stream) {
  return a.NQ == 1 ? launch_decode_kv<D, 1>(a, kv_dtype, stream) : launch_decode_kv<D, 2>(a, kv_dtype, stream);
}

hipError_t launch_decode(const DecodeArgs& a, int D, int kv_dtype, hipStream_t stream) {
  switch (D) {
    case 16:
      return launch_decode_d<16>(a, kv_dtype, stream);
    case 32:
      return launch_decode_d<32>(a, kv_dtype, stream);
    case 64:
      return launch_decode_d<64>(a, kv_dtype, stream);
    case 128:
      return launch_decode_d<128>(a, kv_dtype, stream);
    case 256:
      return launch_decode_d<256>(a, kv_dtype, stream);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace sps
