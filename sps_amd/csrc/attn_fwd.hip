// Forward attention (document-masked causal and SPS sliding-window), bf16/f16 MFMA, gfx950.
//
// One workgroup = 4 waves = 128 query positions; each wave owns 32 queries. Per 32-key block the
// wave computes S^T = K Q^T with v_mfma_f32_32x32x16 (K rows from LDS, Q held in registers), so
// every lane owns one query column: the online-softmax state is lane-local and row reductions need a
// single permlane32 swap. O^T += V^T P^T takes V^T fragments straight out of the row-major LDS
// tile with ds_read_b64_tr_b16 and P^T from the score accumulator converted to 16-bit pairs in
// place.
//
// Schedule: the workgroup's key blocks are the union of its lanes' visible intervals (one range of
// 32-row blocks per key stream, computed once from the prepass's run starts), and each wave
// classifies each block from four numbers (attn_sched.hpp), so no per-block lookups go to memory.
// K/V blocks flow global -> registers -> LDS through a ring of R register sets: a block's loads are
// issued R blocks before it is computed, the LDS tiles are double-buffered, one barrier per block.
//
// Softmax: exp2 domain with log2(e) folded into the scale; the running max is only raised (and the
// accumulator rescaled) when a block's max exceeds it by more than 2^8, so P stays <= 256 and most
// blocks skip the rescale; row sums of P use v_dot2 on the packed 16-bit P the MFMA consumes.
//
// Reference semantics: _attn_fwd_sps / _attn_fwd_inner_sps (triton_sps_flash_attention.py:26-269),
// _attn_fwd (triton_reverse_sps_flash_attention.py:242-331, triton_full_flash_attention.py:204-283):
// P is rounded to the input type before the PV product; LSE = m + log2(l) is saved for the backward.
#include "attn_tiles.hpp"

namespace sps {

constexpr float kRescaleThreshold = 8.0f;

template <int D, class E, int R>
__global__ __launch_bounds__(256) void attn_fwd_kernel(const AttnArgs a) {
  using G = TileGeom<D>;
  static_assert(R % 2 == 0, "the register ring depth must be even (static LDS buffer indices)");
  __shared__ __attribute__((aligned(16))) uint16_t sK[2][G::ELEMS];
  __shared__ __attribute__((aligned(16))) uint16_t sV[2][G::ELEMS];
  __shared__ int s_span[4 * kWaves];

  const MaskSpec m = a.m;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, c32 = lane & 31;
  int b, h, qt;
  q_workgroup(a, b, h, qt);
  const RowView row = row_view(a, b);
  const int qp = qt * kTile + wave * kBlock + c32;
  const bool qvalid = qp < m.N;
  QState st;
  q_setup(a, row, qp, s_span, st);
  const QPlan& plan = st.plan;
  const int nb = plan.count();
  const bool exact = row.mono;
  const int64_t dq_doc = (!exact && qvalid) ? load_doc(a, b, qp) : 0;

  const uint16_t* kbase = a.k + b * a.sk.b + h * a.sk.h;
  const uint16_t* vbase = a.v + b * a.sv.b + h * a.sv.h;

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

  zero_pad_cols<D>(sK[0], tid);
  zero_pad_cols<D>(sK[1], tid);
  zero_pad_cols<D>(sV[0], tid);
  zero_pad_cols<D>(sV[1], tid);

  TileRegs<D> rk[R], rv[R];
  auto issue = [&](int i, TileRegs<D>& tk, TileRegs<D>& tv) {
    const int s = plan.stream(i);
    const int pos0 = stream_pos(m, s, plan.first(i));
    const int step = s == STREAM_NATURAL ? 1 : 2;
    tk.load(kbase, a.sk.n, m.N, tid, pos0, step);
    tv.load(vbase, a.sv.n, m.N, tid, pos0, step);
  };

#pragma unroll
  for (int j = 0; j < R; ++j)
    if (j < nb) issue(j, rk[j], rv[j]);
  if (nb > 0) {
    rk[0].store(sK[0], tid);
    rv[0].store(sV[0], tid);
  }
  if (R < nb) issue(R, rk[0], rv[0]);
  __syncthreads();

  float m_run = -INFINITY, l_run = 0.f;
  f32x16_t acc[G::DC];
#pragma unroll
  for (int dc = 0; dc < G::DC; ++dc) acc[dc] = f32x16_t{};

  vmem_wait_all();
  // Two copies of the loop: exact interval masks (ids non-decreasing), or interval + id checks.
  auto run = [&](auto exact_tag) {
    constexpr bool EXACT = decltype(exact_tag)::value;
    for (int i0 = 0; i0 < nb; i0 += R) {
#pragma unroll
      for (int u = 0; u < R; ++u) {
        const int i = i0 + u;
        if (i < nb) {
          const int nslot = (u + 1) % R;
          if (i + 1 < nb) {
            rk[nslot].store(sK[(u + 1) & 1], tid);
            rv[nslot].store(sV[(u + 1) & 1], tid);
          }
          if (i + 1 + R < nb) issue(i + 1 + R, rk[nslot], rv[nslot]);

          const bool s0 = i < plan.n0;
          const int t0 = plan.first(i);
          const WaveSpan ws = s0 ? st.w0 : st.w1;
          const Interval lr = s0 ? st.r0 : st.r1;
          const int cls = classify_block(ws, t0, EXACT);
          if (cls != TILE_SKIP) {
            const uint16_t* tK = sK[u & 1];
            const uint16_t* tV = sV[u & 1];
            f32x16_t sc = {};
#pragma unroll
            for (int c = 0; c < D / 16; ++c)
              sc = E::mfma(lds_read_b128(tK + c32 * G::RS + 16 * c + 8 * g), qf[c], sc);
            if (cls == TILE_PARTIAL) {
              if constexpr (EXACT) {
                mask_outside(sc, lr.lo, lr.hi, t0, g);
              } else {
                const uint32_t bits = qs_exact_bits(a, b, lr, plan.stream(i), t0, g, dq_doc);
#pragma unroll
                for (int e = 0; e < 16; ++e) sc[e] = ((bits >> e) & 1u) ? sc[e] : -INFINITY;
              }
            }
            float mx = fmaxf(fmaxf(sc[0], sc[1]), sc[2]);
#pragma unroll
            for (int e = 3; e < 15; e += 2) mx = fmaxf(fmaxf(mx, sc[e]), sc[e + 1]);
            mx = fmaxf(mx, sc[15]);
            const float mb = half_max(mx) * a.scale2;
            const bool need = mb > m_run + kRescaleThreshold;
            if (wave_any(need)) {
              const float alpha = need ? fast_exp2(m_run - mb) : 1.f;
              m_run = need ? mb : m_run;
              l_run *= alpha;
#pragma unroll
              for (int dc = 0; dc < G::DC; ++dc) acc[dc] *= alpha;
            }
            const float mu = m_run == -INFINITY ? 0.f : m_run;
            uint32_t pk[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
              const float p0 = fast_exp2(fmaf(sc[2 * j], a.scale2, -mu));
              const float p1 = fast_exp2(fmaf(sc[2 * j + 1], a.scale2, -mu));
              pk[j] = E::pack2(p0, p1);
              l_run = E::sum2(pk[j], l_run);
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
          __syncthreads();
        }
      }
    }
  };
  if (exact)
    run(std::true_type{});
  else
    run(std::false_type{});

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
    if (g == 0) a.lse[((int64_t)b * a.H + h) * m.N + qp] = l_tot > 0.f ? m_run + __log2f(l_tot) : -INFINITY;
  }
}

// Writes the visibility mask exactly as the query-stationary kernels (forward, dQ) evaluate it:
// same plan, same per-wave classification, same per-element tests and lane layout.
__global__ __launch_bounds__(256) void mask_dump_q_kernel(const AttnArgs a) {
  __shared__ int s_span[4 * kWaves];
  const MaskSpec m = a.m;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, c32 = lane & 31;
  int b, h, qt;
  q_workgroup(a, b, h, qt);
  const RowView row = row_view(a, b);
  const int qp = qt * kTile + wave * kBlock + c32;
  const bool qvalid = qp < m.N;
  QState st;
  q_setup(a, row, qp, s_span, st);
  const QPlan& plan = st.plan;
  const bool exact = row.mono;
  const int64_t dq_doc = (!exact && qvalid) ? load_doc(a, b, qp) : 0;
  uint8_t* mrow = a.mask_out + ((int64_t)b * m.N + (qvalid ? qp : 0)) * m.N;
  for (int i = 0; i < plan.count(); ++i) {
    const bool s0 = i < plan.n0;
    const int t0 = plan.first(i), stream = plan.stream(i);
    const WaveSpan ws = s0 ? st.w0 : st.w1;
    const Interval lr = s0 ? st.r0 : st.r1;
    const int cls = classify_block(ws, t0, exact);
    if (cls == TILE_SKIP || !qvalid) continue;
    uint32_t bits = 0xffffu;
    if (cls == TILE_PARTIAL)
      bits = exact ? interval_keep_bits(lr.lo, lr.hi, t0, g) : qs_exact_bits(a, b, lr, stream, t0, g, dq_doc);
    for (int e = 0; e < 16; ++e) {
      if ((bits >> e) & 1u) mrow[stream_pos(m, stream, t0 + acc_row(e, g))] = 1;
    }
  }
}

template <int D, class E>
static hipError_t launch_fwd_t(const AttnArgs& a, hipStream_t stream) {
  const int64_t nblocks = (int64_t)q_tiles(a.m.N) * a.B * a.H;
  if (nblocks == 0) return hipSuccess;
  hipLaunchKernelGGL((attn_fwd_kernel<D, E, 2>), dim3((unsigned)nblocks), dim3(256), 0, stream, a);
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
  const int n = q_tiles(a.m.N) * a.B * a.H;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(mask_dump_q_kernel, dim3(n), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace sps
