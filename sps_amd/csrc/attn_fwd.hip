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
// 32-row blocks per key stream; with documents the prepass writes it into the workgroup's plan),
// and each wave classifies each block from
// four numbers (attn_sched.hpp), so no per-block lookups go to memory.
// K/V blocks are consumed in pairs (64 rows, one barrier per pair) from double-buffered LDS tiles,
// loaded one pair ahead: at head dims of 64 and more by direct global -> LDS loads into dense
// swizzled tiles (run_groups_dma), below through registers into padded tiles (run_pairs). Rows past
// the end of the sequence read as zeros.
//
// Softmax: exp2 domain. The score MFMAs deliver S = K Q^T in fp32 from the unscaled inputs, and one
// FMA per score forms S * scale2 - m_run in fp32 (scale2 = sm_scale * log2 e), as the reference
// scales its fp32 scores (triton_sps_flash_attention.py:78-79): scaling an input operand instead would
// round Q * scale to the input type, an error that grows with the score magnitude. Masked scores are
// set to -inf while still raw, and the running max is taken over the raw scores (times scale2), so
// scale2 must be positive: a negative sm_scale flips the sign bits of Q instead (exact in 16 bits),
// and a zero one is replaced by 2^-100 (every visible score then scales to within 2^-80 of 0, while
// masked ones stay -inf). The running max is only raised (and the accumulator rescaled) when a
// block's max exceeds it by more than 2^8, so P stays <= 256 and most blocks skip the rescale; row
// sums of P use v_dot2 on the packed 16-bit P the MFMA consumes.
//
// Reference semantics: _attn_fwd_sps / _attn_fwd_inner_sps (triton_sps_flash_attention.py:26-269),
// _attn_fwd (triton_reverse_sps_flash_attention.py:242-331, triton_full_flash_attention.py:204-283):
// P is rounded to the input type before the PV product; LSE = m + log2(l) is saved for the backward.
#include "attn_tiles.hpp"

namespace sps {

// Pairs of blocks whose loads are in flight while a pair is computed (run_pairs).
constexpr int kLook = 1;

constexpr float kRescaleThreshold = 8.0f;

// Byte offset past every buffer's range (the host keeps each head slice below 2^31 bytes): a block
// loaded from here reads as zeros.
constexpr uint32_t kOutOfRange = 0x80000000u;

// Waves per SIMD the forward is compiled for. At D = 64 the SPS families run four (their per-wave
// loops are short, so more resident waves hide more of each workgroup's setup: C3 forward -5 %
// against three), full attention three (four measured +4 % at C2, whose longer loops gain less
// from it than they lose to the tighter register budget).
template <int D>
constexpr int fwd_waves_full() {
  return D <= 64 ? 3 : (D <= 128 ? 2 : 1);
}
template <int D>
constexpr int fwd_waves_sps() {
  return D == 64 ? 4 : fwd_waves_full<D>();
}

template <int D, class E, int W>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(W, 8))) void attn_fwd_kernel(const AttnArgs a) {
  using G = TileGeom<D>;
  // Head dims of 64 and more stage K / V blocks by direct global -> LDS loads into dense swizzled
  // tiles (no staging registers, no LDS write instructions); smaller ones through registers into
  // padded tiles.
  constexpr bool kDma = D >= 64;
  using DT = DmaTile<kDma ? D : 64, false>;
  constexpr int TE = kDma ? DT::ELEMS : G::ELEMS;
  // One array per buffer ([block of the pair]): every use names its buffer with a compile-time
  // index, so the compiler can tell the buffers apart, and the score-tile reads of one buffer do not
  // wait for the direct-to-LDS loads still filling the other (measured: -2 % at D = 64, -8 % at
  // D = 128 against register staging).
  __shared__ __attribute__((aligned(16))) uint16_t sK0[2][TE], sK1[2][TE];
  __shared__ __attribute__((aligned(16))) uint16_t sV0[2][TE], sV1[2][TE];
  auto tK = [&](int buf, int y) -> uint16_t* { return buf ? sK1[y] : sK0[y]; };
  auto tV = [&](int buf, int y) -> uint16_t* { return buf ? sV1[y] : sV0[y]; };
  __shared__ int s_span[4 * kWaves];

  const MaskSpec m = a.m;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, c32 = lane & 31;
  int b, h;
  TilePlan tp;
  q_workgroup(a, b, h, tp);
  const RowView row = row_view(a, b, tp.mono);
  const int qp = tp.tile * kTile + wave * kBlock + c32;
  const bool qvalid = qp < m.N;
  QState st;
  int run_start;
  const bool planned = q_begin(a, tp, row, qp, s_span, st, run_start);
  const QPlan& plan = st.plan;
  const int nb = plan.count();
  const bool exact = row.mono;
  const int64_t dq_doc = (!exact && qvalid) ? load_doc(a, b, qp) : 0;

  const BufRsrc k_src = head_rsrc<D>(a.k + b * a.sk.b + h * a.sk.h, a.sk.n, m.N);
  const BufRsrc v_src = head_rsrc<D>(a.v + b * a.sv.b + h * a.sv.h, a.sv.n, m.N);
  const int step = m.family == FAMILY_FULL ? 1 : 2;  // positions between consecutive stream rows
  const auto k_off = TileRegs<D>::offsets(tid, (uint32_t)(step * a.sk.n * 2));
  const auto v_off = TileRegs<D>::offsets(tid, (uint32_t)(step * a.sv.n * 2));

  // Scores are masked (-inf) before they are scaled, and the pair's max is taken over the raw
  // scores, so the scale must be positive: a negative sm_scale flips the sign of Q instead (exact in
  // bf16/f16: S * scale2 = (-S) * (-scale2)), and a zero one becomes 2^-100 (every visible score
  // scales to within 2^-80 of 0, as with scale 0, while masked ones stay -inf).
  const bool flip_q = a.scale2 < 0.f;
  const float scale2 = flip_q ? -a.scale2 : (a.scale2 == 0.f ? 0x1p-100f : a.scale2);

  // Q fragments: B operand of S^T = K Q^T (lane: query c32, d = 16c + 8g .. +7).
  u32x4_t qf[D / 16];
  {
    const uint16_t* qrow = a.q + b * a.sq.b + h * a.sq.h + (int64_t)(qvalid ? qp : 0) * a.sq.n;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      u32x4_t z = {0u, 0u, 0u, 0u};
      qf[c] = qvalid ? *reinterpret_cast<const u32x4_t*>(qrow + 16 * c + 8 * g) : z;
    }
    if (flip_q) {
#pragma unroll
      for (int c = 0; c < D / 16; ++c) qf[c] ^= 0x80008000u;
    }
  }

  if constexpr (!kDma) {
#pragma unroll
    for (int x = 0; x < 2; ++x) {
#pragma unroll
      for (int y = 0; y < 2; ++y) {
        zero_pad_cols<D>(tK(x, y), tid);
        zero_pad_cols<D>(tV(x, y), tid);
      }
    }
  }

  // Byte offset of block i's first row: i * (bytes per block) + a per-stream constant.
  const uint32_t k_blk = (uint32_t)(kBlock * step * a.sk.n * 2), v_blk = (uint32_t)(kBlock * step * a.sv.n * 2);
  const int c0 = stream_pos(m, plan.stream0, kBlock * plan.b0);
  const int c1 = m.family == FAMILY_FULL ? 0 : stream_pos(m, STREAM_TEMPORARY, kBlock * plan.b1) - kBlock * step * plan.n0;
  const uint32_t k_c0 = (uint32_t)(c0 * a.sk.n * 2), k_c1 = (uint32_t)(c1 * a.sk.n * 2);
  const uint32_t v_c0 = (uint32_t)(c0 * a.sv.n * 2), v_c1 = (uint32_t)(c1 * a.sv.n * 2);

  TileRegs<D> rk[kLook][2], rv[kLook][2];
  auto issue = [&](int j, int slot) {
#pragma unroll
    for (int y = 0; y < 2; ++y) {
      const int i = 2 * j + y;
      if (i < nb) {
        const bool s0 = i < plan.n0;
        rk[slot][y].load(k_src, (uint32_t)i * k_blk + (s0 ? k_c0 : k_c1), k_off, tid);
        rv[slot][y].load(v_src, (uint32_t)i * v_blk + (s0 ? v_c0 : v_c1), v_off, tid);
      } else {
        rk[slot][y].zero();
        rv[slot][y].zero();
      }
    }
  };
  auto put = [&](int slot, int buf) {
#pragma unroll
    for (int y = 0; y < 2; ++y) {
      rk[slot][y].store(tK(buf, y), tid);
      rv[slot][y].store(tV(buf, y), tid);
    }
  };
  // LDS-DMA staging. The second block of a last pair that has only one reads as zeros: its scores
  // are masked, and its V rows must be finite for the zero-weighted PV product.
  const auto k_dma = DT::sources(tid, (uint32_t)(step * a.sk.n * 2));
  const auto v_dma = DT::sources(tid, (uint32_t)(step * a.sv.n * 2));
  auto issue_dma = [&](int j, int buf) {
#pragma unroll
    for (int y = 0; y < 2; ++y) {
      const int i = 2 * j + y;
      const bool s0 = i < plan.n0, in = i < nb;
      DT::load(k_src, in ? (uint32_t)i * k_blk + (s0 ? k_c0 : k_c1) : kOutOfRange, k_dma, tK(buf, y), wave);
      DT::load(v_src, in ? (uint32_t)i * v_blk + (s0 ? v_c0 : v_c1) : kOutOfRange, v_dma, tV(buf, y), wave);
    }
  };
  // Fragment reads of a staged key block.
  auto row_frag = [&](const uint16_t* tile, int c) {
    if constexpr (kDma)
      return lds_read_b128(tile + DT::frag(c32, g, c));
    else
      return lds_read_b128(tile + c32 * G::RS + 16 * c + 8 * g);
  };
  auto tr_frag = [&](const uint16_t* tile, int kh, int dc) {
    if constexpr (kDma)
      return DT::frag_tr(tile, 16 * kh, dc, lane);
    else
      return lds_frag_tr(tile, G::RS, 16 * kh, 32 * dc, lane);
  };
  // With LDS-DMA staging the first pair's loads cost no registers: they go out now, ahead of the
  // lanes' setup.
  if constexpr (kDma)
    if (nb > 0) issue_dma(0, 0);

  if (planned) q_lanes(m, qp, run_start, st);
  float negm = 0.f;  // -m_run (0 while no score has been seen): the per-score FMA subtracts m_run
  float m_run = -INFINITY, l_run[4] = {0.f, 0.f, 0.f, 0.f};
  // The rescale test in raw-score units: a pair's raw max above thr = (m_run + threshold) / scale2
  // (any finite score while none has been seen) raises m_run, so the test is one compare per pair.
  float thr = -INFINITY;
  const float inv_scale2 = 1.f / scale2;
  f32x16_t acc[G::DC];
#pragma unroll
  for (int dc = 0; dc < G::DC; ++dc) acc[dc] = f32x16_t{};

  // One pair = two 32-row key blocks staged together (one barrier per pair); the softmax runs block
  // by block (score tile, mask if partial, max / rescale decision, exponentials and PV), so only one
  // 16-register score tile is live: against both tiles and one joint decision per pair, 40 fewer
  // VGPRs, which is what lets D = 64 run four waves per SIMD.
  auto run = [&](auto exact_tag) {
    constexpr bool EXACT = decltype(exact_tag)::value;
    auto cls_of = [&](int i) {
      return classify_block(i < plan.n0 ? st.w0 : st.w1, plan.first(i), EXACT);
    };
    const BlockMask bm = q_block_mask(st, EXACT);
    auto body = [&](int j, int buf) {
      int act2, full2;
      pair_codes(bm, 2 * j, nb, cls_of, act2, full2);
      if (act2 == 0) return;
#pragma unroll
      for (int y = 0; y < 2; ++y) {
        if (!((act2 >> y) & 1)) continue;
        const uint16_t* kt = tK(buf, y);
        f32x16_t sc = E::mfma(row_frag(kt, 0), qf[0], f32x16_t{});
#pragma unroll
        for (int c = 1; c < D / 16; ++c) sc = E::mfma(row_frag(kt, c), qf[c], sc);
        if (!((full2 >> y) & 1)) {
          const int i = 2 * j + y;
          const bool s0 = i < plan.n0;
          const int t0 = plan.first(i);
          const Interval lr = s0 ? st.r0 : st.r1;
          mask_partial<EXACT>(sc, lr, s0 ? st.w0 : st.w1, t0, g,
                              [&] { return qs_exact_bits(a, b, lr, plan.stream(i), t0, g, dq_doc); });
        }
        // The block's max of the raw scores (scaled units: times scale2 > 0). m_run is raised only
        // past the lazy-rescale threshold; the scores themselves stay raw, so a rescale touches only
        // the accumulators, and they are scaled below by one FMA each, S * scale2 - m_run, in fp32.
        float mx = max3f(sc[0], sc[1], sc[2]);
#pragma unroll
        for (int e = 3; e < 15; e += 2) mx = max3f(mx, sc[e], sc[e + 1]);
        mx = __builtin_elementwise_maximum(mx, sc[15]);
        const float raw = half_max(mx);
        const bool need = raw > thr;
        if (wave_any(need)) {
          const float mb = raw * scale2;
          const float m_new = need ? mb : m_run;
          const float alpha = need ? fast_exp2(m_run - m_new) : 1.f;
          // While no lane has seen a score the sums and accumulators are still zero: nothing to scale.
          if (wave_any(m_run != -INFINITY)) {
#pragma unroll
            for (int r = 0; r < 4; ++r) l_run[r] *= alpha;
#pragma unroll
            for (int dc = 0; dc < G::DC; ++dc) acc[dc] *= alpha;
          }
          m_run = m_new;
          negm = m_run == -INFINITY ? 0.f : -m_run;
          thr = m_run == -INFINITY ? -INFINITY : (m_run + kRescaleThreshold) * inv_scale2;
        }
        uint32_t pk[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float p0 = fast_exp2(__builtin_fmaf(sc[2 * e], scale2, negm));
          const float p1 = fast_exp2(__builtin_fmaf(sc[2 * e + 1], scale2, negm));
          pk[e] = E::pack2(p0, p1);
          l_run[e & 3] = E::sum2(pk[e], l_run[e & 3]);  // four independent partial sums
        }
        const uint16_t* vt = tV(buf, y);
#pragma unroll
        for (int dc = 0; dc < G::DC; ++dc) {
#pragma unroll
          for (int kh = 0; kh < 2; ++kh) {
            const u32x4_t pf = {pk[4 * kh], pk[4 * kh + 1], pk[4 * kh + 2], pk[4 * kh + 3]};
            acc[dc] = E::mfma(tr_frag(vt, kh, dc), pf, acc[dc]);
          }
        }
      }
    };
    if constexpr (kDma)
      run_groups_dma<2, true>(nb, issue_dma, body);
    else
      run_pairs<kLook>(nb, issue, put, body);
  };
  if (exact)
    run(std::true_type{});
  else
    run(std::false_type{});

  // Epilogue: combine the two halves' partial sums, normalise, store O (lane = query row) and LSE.
  const float l_tot = half_sum((l_run[0] + l_run[1]) + (l_run[2] + l_run[3]));
  // 1 / l with the hardware reciprocal (1 ulp): the division sequence cost ~10 VALU per wave.
  const float inv = l_tot > 0.f ? __builtin_amdgcn_rcpf(l_tot) : 0.f;
  uint16_t* orow = a.out + b * a.sout.b + h * a.sout.h + (int64_t)(qvalid ? qp : 0) * a.sout.n;
  auto piece = [&](int dc, int ii) {
    return u32x2_t{E::pack2(acc[dc][4 * ii] * inv, acc[dc][4 * ii + 1] * inv),
                   E::pack2(acc[dc][4 * ii + 2] * inv, acc[dc][4 * ii + 3] * inv)};
  };
  // With dense tiles and 16-byte aligned rows, O goes through the wave's idle LDS tile so every
  // global store writes whole rows.
  bool staged = false;
  if constexpr (kDma) {
    if (rows16_ok(a.out, a.sout)) {
      const int q0 = tp.tile * kTile + wave * kBlock;
      store_rows_via_lds<D>(tK(wave >> 1, wave & 1), lane, a.out + b * a.sout.b + h * a.sout.h + (int64_t)q0 * a.sout.n,
                            a.sout.n, imin(kBlock, m.N - q0), piece);
      staged = true;
    }
  }
  if (qvalid) {
    if (!staged) {
#pragma unroll
      for (int dc = 0; dc < G::DC; ++dc) {
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          const int d0 = 32 * dc + 8 * ii + 4 * g;
          if (d0 < D) *reinterpret_cast<u32x2_t*>(orow + d0) = piece(dc, ii);
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
  int b, h;
  TilePlan tp;
  q_workgroup(a, b, h, tp);
  const RowView row = row_view(a, b, tp.mono);
  const int qp = tp.tile * kTile + wave * kBlock + c32;
  const bool qvalid = qp < m.N;
  QState st;
  int run_start;
  if (q_begin(a, tp, row, qp, s_span, st, run_start)) q_lanes(m, qp, run_start, st);
  const QPlan& plan = st.plan;
  const bool exact = row.mono;
  const int64_t dq_doc = (!exact && qvalid) ? load_doc(a, b, qp) : 0;
  uint8_t* mrow = a.mask_out + ((int64_t)b * m.N + (qvalid ? qp : 0)) * m.N;
  const BlockMask bm = q_block_mask(st, exact);
  for (int i = 0; i < plan.count(); ++i) {
    const bool s0 = i < plan.n0;
    const int t0 = plan.first(i), stream = plan.stream(i);
    const WaveSpan ws = s0 ? st.w0 : st.w1;
    const Interval lr = s0 ? st.r0 : st.r1;
    const int cls = i < 128 ? mask_class(bm, i) : classify_block(ws, t0, exact);
    if (cls == TILE_SKIP || !qvalid) continue;
    uint32_t bits = 0xffffu;
    if (cls == TILE_PARTIAL) {
      f32x16_t z = {};
      auto exact_bits = [&] { return qs_exact_bits(a, b, lr, stream, t0, g, dq_doc); };
      if (exact)
        mask_partial<true>(z, lr, ws, t0, g, exact_bits);
      else
        mask_partial<false>(z, lr, ws, t0, g, exact_bits);
      bits = 0;
      for (int e = 0; e < 16; ++e) bits |= (uint32_t)(z[e] == 0.f) << e;
    }
    for (int e = 0; e < 16; ++e) {
      if ((bits >> e) & 1u) mrow[stream_pos(m, stream, t0 + acc_row(e, g))] = 1;
    }
  }
}

template <int D, class E>
static hipError_t launch_fwd_t(const AttnArgs& a, hipStream_t stream) {
  const int64_t nblocks = (int64_t)q_tiles(a.m.N) * a.B * a.H;
  if (nblocks == 0) return hipSuccess;
  if (a.m.family == FAMILY_FULL)
    hipLaunchKernelGGL((attn_fwd_kernel<D, E, fwd_waves_full<D>()>), dim3((unsigned)nblocks), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((attn_fwd_kernel<D, E, fwd_waves_sps<D>()>), dim3((unsigned)nblocks), dim3(256), 0, stream, a);
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
    SPS_FWD_CASE(256)
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
