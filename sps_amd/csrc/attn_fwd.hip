// Forward attention (document-masked causal and SPS sliding-window), bf16/f16 MFMA, gfx950.
//
// One workgroup = 4 waves = 128 query positions; each wave owns 32 queries. Per 32-key block the
// wave computes S^T = K Q^T with v_mfma_f32_32x32x16 (K rows from LDS, Q held in registers), so
// every lane owns one query column: the online-softmax state (running max, running sum, rescale
// factor) is lane-local and the row reductions need a single permlane32 swap. O^T += V^T P^T
// takes V^T fragments straight out of the row-major LDS tile with ds_read_b64_tr_b16 and P^T from
// the score accumulator converted to 16-bit pairs in place. K/V tiles are double-buffered in LDS
// with one barrier per block; the next block's global loads are in flight during the MFMAs.
//
// Reference semantics: _attn_fwd_sps / _attn_fwd_inner_sps (triton_sps_flash_attention.py:26-269),
// _attn_fwd (triton_reverse_sps_flash_attention.py:242-331, triton_full_flash_attention.py:204-283):
// exp2-domain online softmax with the scale folded into log2(e); P is rounded to the input type
// before the PV product; LSE = m + log2(l) is saved for the backward pass.
#include "attn_tiles.hpp"

namespace sps {

__global__ void doc_granules_kernel(const AttnArgs a) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= a.B * a.NG) return;
  const int b = idx / a.NG, gi = idx - b * a.NG;
  const int lo = gi * kGranule;
  const int hi = lo + kGranule < a.m.N ? lo + kGranule : a.m.N;
  int64_t mn = INT64_MAX, mx = INT64_MIN;
  for (int p = lo; p < hi; ++p) {
    const int64_t d = load_doc(a, b, p);
    mn = d < mn ? d : mn;
    mx = d > mx ? d : mx;
  }
  a.gmin[idx] = mn;
  a.gmax[idx] = mx;
}

template <int D, class E>
__global__ __launch_bounds__(256) void attn_fwd_kernel(const AttnArgs a) {
  using G = TileGeom<D>;
  __shared__ __attribute__((aligned(16))) uint16_t sK[2][G::ELEMS];
  __shared__ __attribute__((aligned(16))) uint16_t sV[2][G::ELEMS];
  __shared__ int64_t sDoc[2][kBlock];

  const MaskSpec m = a.m;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, c32 = lane & 31;

  const int nqt = (m.N + kTile - 1) / kTile;
  const int lid = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = lid / nqt;
  const int qt = nqt - 1 - (lid - bh * nqt);  // later (heavier) query tiles first
  const int b = bh / a.H, h = bh - b * a.H;
  const int qa = qt * kTile;
  const int qw = qa + wave * kBlock;
  const int qp = qw + c32;
  const bool qvalid = qp < m.N;

  const uint16_t* kbase = a.k + b * a.sk.b + h * a.sk.h;
  const uint16_t* vbase = a.v + b * a.sv.b + h * a.sv.h;
  const int64_t* gmin = a.gmin + (int64_t)b * a.NG;
  const int64_t* gmax = a.gmax + (int64_t)b * a.NG;

  // Q fragments: B operand of S^T = K Q^T (lane: query c32, d = 16c + 8g .. +7).
  u32x4_t qf[D / 16];
  {
    const uint16_t* qrow = a.q + b * a.sq.b + h * a.sq.h + (int64_t)(qvalid ? qp : 0) * a.sq.n;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      u32x4_t z = {0u, 0u, 0u, 0u};
      qf[c] = qvalid ? *reinterpret_cast<const u32x4_t*>(qrow + 16 * c + 8 * g) : z;
    }
  }
  const int64_t dq = (m.has_docs && qvalid) ? load_doc(a, b, qp) : 0;

  const QSchedule s = make_qschedule(m, qa);
  const int nb = s.n0 + s.n1;
  const int wg_qhi = qa + kTile - 1 < m.N - 1 ? qa + kTile - 1 : m.N - 1;
  const int w_qhi = qw + kBlock - 1 < m.N - 1 ? qw + kBlock - 1 : m.N - 1;
  DocRange wg_qd = {0, 0}, w_qd = {0, 0};
  if (m.has_docs) {
    wg_qd = doc_range(gmin, gmax, qa, wg_qhi);
    if (qw < m.N) w_qd = doc_range(gmin, gmax, qw, w_qhi);
  }

  zero_pad_cols<D>(sK[0], tid);
  zero_pad_cols<D>(sK[1], tid);
  zero_pad_cols<D>(sV[0], tid);
  zero_pad_cols<D>(sV[1], tid);

  TileRegs<D> rk, rv;
  int64_t rdoc = 0;
  auto load_block = [&](const KeyRun& kr) {
    auto pos = [&](int r) { return key_pos(m, kr, r); };
    rk.load(kbase, a.sk.n, m.N, tid, pos);
    rv.load(vbase, a.sv.n, m.N, tid, pos);
    if (m.has_docs && tid < kBlock) {
      const int kp = pos(tid);
      rdoc = kp < m.N ? load_doc(a, b, kp) : INT64_MIN;
    }
  };
  auto store_block = [&](int buf) {
    rk.store(sK[buf], tid);
    rv.store(sV[buf], tid);
    if (m.has_docs && tid < kBlock) sDoc[buf][tid] = rdoc;
  };

  float m_run = -INFINITY, l_run = 0.f;
  f32x16_t acc[G::DC];
#pragma unroll
  for (int dc = 0; dc < G::DC; ++dc) acc[dc] = f32x16_t{};

  int cur = qs_next_block(m, s, qa, wg_qhi, wg_qd, gmin, gmax, -1);
  KeyRun kr_cur = qschedule_block(s, cur < nb ? cur : 0);
  if (cur < nb) {
    load_block(kr_cur);
    store_block(0);
  }
  __syncthreads();
  int buf = 0;
  while (cur < nb) {
    const int nxt = qs_next_block(m, s, qa, wg_qhi, wg_qd, gmin, gmax, cur);
    const KeyRun kr_nxt = qschedule_block(s, nxt < nb ? nxt : 0);
    if (nxt < nb) load_block(kr_nxt);

    const int cls = classify(m, qw, w_qhi, kr_cur, w_qd, run_docs(m, kr_cur, gmin, gmax));
    if (cls != TILE_SKIP) {
      const uint16_t* tK = sK[buf];
      const uint16_t* tV = sV[buf];
      f32x16_t sc = {};
#pragma unroll
      for (int c = 0; c < D / 16; ++c)
        sc = E::mfma(lds_read_b128(tK + c32 * G::RS + 16 * c + 8 * g), qf[c], sc);
      if (cls == TILE_PARTIAL) {
        const uint32_t bits = qs_mask_bits(m, qp, dq, kr_cur, g, sDoc[buf]);
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (!((bits >> i) & 1u)) sc[i] = -INFINITY;
      }
      float mx = sc[0];
#pragma unroll
      for (int i = 1; i < 16; ++i) mx = fmaxf(mx, sc[i]);
      mx = half_max(mx);
      const float m_new = fmaxf(m_run, mx * a.scale2);
      const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = fast_exp2(m_run - m_use);
      float rs = 0.f;
      uint32_t pk[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float p0 = fast_exp2(fmaf(sc[2 * j], a.scale2, -m_use));
        const float p1 = fast_exp2(fmaf(sc[2 * j + 1], a.scale2, -m_use));
        rs += p0 + p1;
        pk[j] = E::pack2(p0, p1);
      }
      l_run = fmaf(l_run, alpha, rs);
      m_run = m_new;
      if (wave_any(alpha != 1.f)) {
#pragma unroll
        for (int dc = 0; dc < G::DC; ++dc) acc[dc] *= alpha;
      }
#pragma unroll
      for (int dc = 0; dc < G::DC; ++dc) {
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
          const u32x4_t pf = {pk[4 * kh], pk[4 * kh + 1], pk[4 * kh + 2], pk[4 * kh + 3]};
          acc[dc] = E::mfma(lds_frag_tr(tV, G::RS, 16 * kh, 32 * dc, lane), pf, acc[dc]);
        }
      }
    }

    if (nxt < nb) store_block(buf ^ 1);
    __syncthreads();
    buf ^= 1;
    cur = nxt;
    kr_cur = kr_nxt;
  }

  // Epilogue: combine the two halves' partial sums, normalise, store O (lane = query row) and LSE.
  const float l_tot = half_sum(l_run);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (qvalid) {
    uint16_t* orow = a.out + b * a.sout.b + h * a.sout.h + (int64_t)qp * a.sout.n;
#pragma unroll
    for (int dc = 0; dc < G::DC; ++dc) {
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int d0 = 32 * dc + 8 * ii + 4 * g;
        if (d0 < D) {
          u32x2_t w = {E::pack2(acc[dc][4 * ii] * inv, acc[dc][4 * ii + 1] * inv),
                       E::pack2(acc[dc][4 * ii + 2] * inv, acc[dc][4 * ii + 3] * inv)};
          *reinterpret_cast<u32x2_t*>(orow + d0) = w;
        }
      }
    }
    if (g == 0) a.lse[(int64_t)bh * m.N + qp] = l_tot > 0.f ? m_run + __log2f(l_tot) : -INFINITY;
  }
}

// Writes the visibility mask exactly as the query-stationary kernels (forward, dQ) evaluate it:
// same block schedule, same per-wave classification, same per-element predicate and lane layout.
__global__ __launch_bounds__(256) void mask_dump_q_kernel(const AttnArgs a) {
  __shared__ int64_t sDoc[kBlock];
  const MaskSpec m = a.m;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, c32 = lane & 31;
  const int nqt = (m.N + kTile - 1) / kTile;
  const int b = blockIdx.x / nqt;
  const int qa = (blockIdx.x - b * nqt) * kTile;
  const int qw = qa + wave * kBlock;
  const int qp = qw + c32;
  const bool qvalid = qp < m.N;
  const int64_t* gmin = a.gmin + (int64_t)b * a.NG;
  const int64_t* gmax = a.gmax + (int64_t)b * a.NG;
  const int64_t dq = (m.has_docs && qvalid) ? load_doc(a, b, qp) : 0;
  const QSchedule s = make_qschedule(m, qa);
  const int nb = s.n0 + s.n1;
  const int wg_qhi = qa + kTile - 1 < m.N - 1 ? qa + kTile - 1 : m.N - 1;
  const int w_qhi = qw + kBlock - 1 < m.N - 1 ? qw + kBlock - 1 : m.N - 1;
  DocRange wg_qd = {0, 0}, w_qd = {0, 0};
  if (m.has_docs) {
    wg_qd = doc_range(gmin, gmax, qa, wg_qhi);
    if (qw < m.N) w_qd = doc_range(gmin, gmax, qw, w_qhi);
  }
  uint8_t* mrow = a.mask_out + ((int64_t)b * m.N + qp) * m.N;
  for (int cur = qs_next_block(m, s, qa, wg_qhi, wg_qd, gmin, gmax, -1); cur < nb;
       cur = qs_next_block(m, s, qa, wg_qhi, wg_qd, gmin, gmax, cur)) {
    const KeyRun kr = qschedule_block(s, cur);
    if (m.has_docs && tid < kBlock) {
      const int kp = key_pos(m, kr, tid);
      sDoc[tid] = kp < m.N ? load_doc(a, b, kp) : INT64_MIN;
    }
    __syncthreads();
    const int cls = classify(m, qw, w_qhi, kr, w_qd, run_docs(m, kr, gmin, gmax));
    if (cls != TILE_SKIP && qvalid) {
      const uint32_t bits = cls == TILE_FULL ? 0xffffu : qs_mask_bits(m, qp, dq, kr, g, sDoc);
      for (int i = 0; i < 16; ++i) {
        const int kp = key_pos(m, kr, acc_row(i, g));
        if ((bits >> i) & 1u) mrow[kp] = 1;
      }
    }
    __syncthreads();
  }
}

hipError_t launch_doc_granules(const AttnArgs& a, hipStream_t stream) {
  const int n = a.B * a.NG;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(doc_granules_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, a);
  return hipGetLastError();
}

template <int D, class E>
static hipError_t launch_fwd_t(const AttnArgs& a, hipStream_t stream) {
  const int nqt = (a.m.N + kTile - 1) / kTile;
  const int64_t nblocks = (int64_t)nqt * a.B * a.H;
  if (nblocks == 0) return hipSuccess;
  hipLaunchKernelGGL((attn_fwd_kernel<D, E>), dim3((unsigned)nblocks), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_attn_fwd(const AttnArgs& a, int D, int is_f16, hipStream_t stream) {
#define SPS_FWD_CASE(DD)                                                                      \
  case DD:                                                                                    \
    return is_f16 ? launch_fwd_t<DD, ElemF16>(a, stream) : launch_fwd_t<DD, ElemBF16>(a, stream);
  switch (D) {
    SPS_FWD_CASE(16)
    SPS_FWD_CASE(32)
    SPS_FWD_CASE(64)
    SPS_FWD_CASE(128)
    default:
      return hipErrorInvalidValue;
  }
#undef SPS_FWD_CASE
}

hipError_t launch_mask_dump_q(const AttnArgs& a, hipStream_t stream) {
  const int nqt = (a.m.N + kTile - 1) / kTile;
  const int n = nqt * a.B;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(mask_dump_q_kernel, dim3(n), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace sps
