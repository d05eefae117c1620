// Backward attention, bf16/f16 MFMA, gfx950. Two deterministic passes, no atomics, as in the
// reference (_sps_bwd_dq_kernel / _sps_bwd_dkdv_kernel, triton_sps_flash_attention.py:272-488;
// reverse twins triton_reverse_sps_flash_attention.py:370-599; full triton_full_flash_attention.py:301-460):
//
//  1. dQ pass (query-stationary, the forward's plan and classification). Its prologue computes
//     Delta = rowsum(O * dO) for its own queries and stores it for pass 2 (this replaces the
//     reference's separate _attn_bwd_preprocess launch). Per 32-key block:
//       S^T = K Q^T, dP^T = V dO^T (K, V rows from LDS; Q, dO in registers),
//       P = exp2(S*scale2 - LSE) (one fp32 FMA per score, as the reference scales its fp32 scores:
//       triton_sps_flash_attention.py:471), dS = P (dP - Delta)   (lane-local LSE and Delta),
//       dQ^T += K^T dS^T  (K^T fragments via ds_read_b64_tr_b16).
//  2. dK/dV pass (key-stationary). A workgroup owns 128 keys of one stream (natural, persistent
//     or temporary), each wave 32 of them held in registers; it walks the 32-query chunks of the
//     union of its lanes' query intervals (persistent keys: diagonal to document end; temporary
//     keys: the w-token window):
//       S = Q K^T, dP = dO V^T (Q, dO rows from LDS; K, V in registers),
//       P = exp2(S*scale2 - LSE) (fp32 FMA per score, triton_sps_flash_attention.py:361),
//       dV^T += dO^T P, dK^T += Q^T dS (dO^T, Q^T fragments via ds_read_b64_tr_b16).
// Both passes consume their tiles in groups of four 32-row blocks (one barrier per group) through
// the run_groups pipeline: buffer loads one group ahead into registers, double-buffered LDS; with
// documents the first group's loads leave right after the workgroup's plan is read. dK and dQ are
// scaled by sm_scale at the end, as in the reference.
#include "attn_tiles.hpp"

namespace sps {

// Groups of blocks whose loads are in flight while a group is computed (run_groups).
constexpr int kLook = 1;

// Blocks per barrier (LDS budget: up to D = 128 both passes run 2 workgroups per CU, so four 32-row
// blocks of two tensors, double-buffered, fit; fewer barriers per block than pairs). At D = 256 a
// block is 16 KiB, so groups of two (128 KiB of tiles, one workgroup per CU).
template <int D>
constexpr int bwd_group() { return D >= 256 ? 2 : 4; }

// One waves-per-SIMD floor per head dim: 2 at D <= 64; above, the MFMA accumulators of D-wide rows
// need the registers of one wave per SIMD.
template <int D>
constexpr int bwd_waves() { return D <= 64 ? 2 : 1; }

// The dQ pass at D = 64 runs 3 waves per SIMD instead: groups of two blocks (32 KiB of tiles, so the
// LDS holds three workgroups per CU) and 168 VGPRs (dQ -4 % at C3, -6 % at C2 against four-block
// groups at 2 waves per SIMD).
template <int D>
constexpr int dq_group() { return D == 64 ? 2 : bwd_group<D>(); }
template <int D>
constexpr int dq_waves() { return D == 64 ? 3 : bwd_waves<D>(); }

// The wave index, wave-uniform at D = 64 (so every LDS address derived from it, the direct-to-LDS
// loads' M0 values among them, is computed in scalar registers instead of VGPRs that the 3-wave dQ
// pass would have to spill).
template <int D>
__device__ __forceinline__ int wave_index() {
  return D == 64 ? wave_uniform((int)threadIdx.x >> 6) : (int)threadIdx.x >> 6;
}

// The wave's own 32-row tile of a [2][NG][32 * D] staging array (an idle buffer at the end of the
// kernel): every layout holds at least kWaves of them.
template <int NG, int TE>
__device__ __forceinline__ uint16_t* wave_tile(uint16_t (&arr)[2][NG][TE], int wave) {
  static_assert(2 * NG >= kWaves, "one tile per wave");
  return &arr[0][0][0] + wave * TE;
}

template <int D, class E>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(dq_waves<D>(), 8))) void attn_bwd_dq_kernel(const AttnArgs a) {
  using G = TileGeom<D>;
  constexpr int NG = dq_group<D>();
  // Head dims of 64 and more stage K / V blocks by direct global -> LDS loads into dense swizzled
  // tiles (frees the staging VGPRs: -7 % at D = 128, -2 % of the C3 step at D = 64 under the
  // iterative ILP schedule); smaller ones through registers into padded tiles.
  constexpr bool kDma = D >= 64;
  // The conflict-free swizzle costs a few address VGPRs: at D = 64 (3 waves per SIMD) and D = 256
  // they would spill, so those keep the register-lean one.
  using DT = DmaTile<kDma ? D : 64, D == 128>;
  constexpr int TE = kDma ? DT::ELEMS : G::ELEMS;
  __shared__ __attribute__((aligned(16))) uint16_t sK[2][NG][TE];  // [buffer][block of the group]
  __shared__ __attribute__((aligned(16))) uint16_t sV[2][NG][TE];
  __shared__ int s_span[4 * kWaves];

  const MaskSpec m = a.m;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_index<D>();
  const int g = lane >> 5, c32 = lane & 31;
  int b, h;
  TilePlan tp;
  q_workgroup(a, b, h, tp);
  const RowView row = row_view(a, b, tp.mono);
  const int qp = tp.tile * kTile + wave * kBlock + c32;
  const bool qvalid = qp < m.N;
  const int qsafe = qvalid ? qp : 0;
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

  // Q, dO and O fragments (B operands; lane: query c32, d = 16c + 8g .. +7) and the LSE, loaded
  // raw here; everything computed from them waits until the first group's loads are issued too.
  u32x4_t qf[D / 16], dof[D / 16], of[D / 16];
  const int64_t rowid = ((int64_t)b * a.H + h) * m.N + qsafe;
  {
    const uint16_t* qrow = a.q + b * a.sq.b + h * a.sq.h + (int64_t)qsafe * a.sq.n;
    const uint16_t* dorow = a.dO + b * a.sdo.b + h * a.sdo.h + (int64_t)qsafe * a.sdo.n;
    const uint16_t* orow = a.o + b * a.so.b + h * a.so.h + (int64_t)qsafe * a.so.n;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      u32x4_t z = {0u, 0u, 0u, 0u};
      qf[c] = qvalid ? *reinterpret_cast<const u32x4_t*>(qrow + 16 * c + 8 * g) : z;
      dof[c] = qvalid ? *reinterpret_cast<const u32x4_t*>(dorow + 16 * c + 8 * g) : z;
      of[c] = qvalid ? *reinterpret_cast<const u32x4_t*>(orow + 16 * c + 8 * g) : z;
    }
  }
  const float lse_raw = qvalid ? a.lse[rowid] : 0.f;

  if constexpr (!kDma) {
#pragma unroll
    for (int x = 0; x < 2; ++x) {
#pragma unroll
      for (int y = 0; y < NG; ++y) {
        zero_pad_cols<D>(sK[x][y], tid);
        zero_pad_cols<D>(sV[x][y], tid);
      }
    }
  }

  // Byte offset of block i's first row: i * (bytes per block) + a per-stream constant (modulo 2^32).
  const uint32_t k_blk = (uint32_t)(kBlock * step * a.sk.n * 2), v_blk = (uint32_t)(kBlock * step * a.sv.n * 2);
  const int c0 = stream_pos(m, plan.stream0, kBlock * plan.b0);
  const int c1 = m.family == FAMILY_FULL ? 0 : stream_pos(m, STREAM_TEMPORARY, kBlock * plan.b1) - kBlock * step * plan.n0;
  const uint32_t k_c0 = (uint32_t)(c0 * a.sk.n * 2), k_c1 = (uint32_t)(c1 * a.sk.n * 2);
  const uint32_t v_c0 = (uint32_t)(c0 * a.sv.n * 2), v_c1 = (uint32_t)(c1 * a.sv.n * 2);

  // Register staging (head dims below 64).
  TileRegs<D> rk[kLook][NG], rv[kLook][NG];
  auto issue_regs = [&](int j, int slot) {
#pragma unroll
    for (int y = 0; y < NG; ++y) {
      const int i = NG * j + y;
      if (i < nb) {
        const bool s0 = i < plan.n0;
        rk[slot][y].load(k_src, (uint32_t)i * k_blk + (s0 ? k_c0 : k_c1), k_off, tid);
        rv[slot][y].load(v_src, (uint32_t)i * v_blk + (s0 ? v_c0 : v_c1), v_off, tid);
      }
    }
  };
  auto put_regs = [&](int slot, int buf) {
#pragma unroll
    for (int y = 0; y < NG; ++y) {
      rk[slot][y].store(sK[buf][y], tid);
      rv[slot][y].store(sV[buf][y], tid);
    }
  };
  // LDS-DMA staging (head dims of 64 and more).
  const auto k_dma = DT::sources(tid, (uint32_t)(step * a.sk.n * 2));
  const auto v_dma = DT::sources(tid, (uint32_t)(step * a.sv.n * 2));
  auto issue_dma = [&](int j, int buf) {
#pragma unroll
    for (int y = 0; y < NG; ++y) {
      const int i = NG * j + y;
      if (i < nb) {
        const bool s0 = i < plan.n0;
        DT::load(k_src, (uint32_t)i * k_blk + (s0 ? k_c0 : k_c1), k_dma, sK[buf][y], wave);
        DT::load(v_src, (uint32_t)i * v_blk + (s0 ? v_c0 : v_c1), v_dma, sV[buf][y], wave);
      }
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
  // With LDS-DMA staging the first group's loads cost no registers: they go out now, with the Q /
  // dO / O fragment loads below, ahead of the lanes' setup.
  if constexpr (kDma) issue_dma(0, 0);

  f32x16_t acc[G::DC];
#pragma unroll
  for (int dc = 0; dc < G::DC; ++dc) acc[dc] = f32x16_t{};

  if (planned) q_lanes(m, qp, run_start, st);

  // Delta = rowsum(O * dO) of the lane's query, stored for the dK/dV pass: one v_dot2 per packed pair
  // (two exact products and the fp32 accumulation in one instruction), two independent partial sums.
  float delta;
  {
    float part[2] = {0.f, 0.f};
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
#pragma unroll
      for (int j = 0; j < 4; ++j) part[j & 1] = E::dot2(of[c][j], dof[c][j], part[j & 1]);
    }
    delta = half_sum(part[0] + part[1]);
  }
  const float lse = lse_raw == -INFINITY ? 0.f : lse_raw;  // a query with no visible key: every score is masked to -inf
  if (qvalid && g == 0) {
    // Seeds of the dK/dV pass for this query: -LSE and -Delta.
    float* seed = a.seeds + ((int64_t)b * a.H + h) * 2 * m.N + qp;
    seed[0] = -lse;
    seed[m.N] = -delta;
  }

  // The dP tile starts from -Delta, so it comes out of the MFMAs as dP - Delta and dS = P * dP' is one
  // VALU operation per element; the S tile is scaled in fp32 (one FMA per score forms
  // S * scale2 - LSE), never by rounding a scaled Q to the input type.
  const float scale2 = a.scale2, neg_lse = -lse;
  const f32x16_t c_dp = f32x16_t{} - delta;

  auto run = [&](auto exact_tag) {
    constexpr bool EXACT = decltype(exact_tag)::value;
    auto cls_of = [&](int i) {
      return classify_block(i < plan.n0 ? st.w0 : st.w1, plan.first(i), EXACT);
    };
    const BlockMask bm = q_block_mask(st, EXACT);
    auto body = [&](int j, int buf) {
      int act2, full2;
      group_codes<NG>(bm, NG * j, nb, cls_of, act2, full2);
#pragma unroll
      for (int y = 0; y < NG; ++y) {
        const int i = NG * j + y;
        const bool s0 = i < plan.n0;
        const int t0 = plan.first(i);
        const WaveSpan ws = s0 ? st.w0 : st.w1;
        const Interval lr = s0 ? st.r0 : st.r1;
        if ((act2 >> y) & 1) {
          const uint16_t* tK = sK[buf][y];
          const uint16_t* tV = sV[buf][y];
          f32x16_t sc = f32x16_t{}, dp = c_dp;
#pragma unroll
          for (int c = 0; c < D / 16; ++c) {
            sc = E::mfma(row_frag(tK, c), qf[c], sc);
            dp = E::mfma(row_frag(tV, c), dof[c], dp);
          }
#pragma unroll
          for (int e = 0; e < 16; ++e) sc[e] = __builtin_fmaf(sc[e], scale2, neg_lse);
          if (!((full2 >> y) & 1))
            mask_partial<EXACT>(sc, lr, ws, t0, g,
                                [&] { return qs_exact_bits(a, b, lr, plan.stream(i), t0, g, dq_doc); });
          uint32_t dsk[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float p0 = fast_exp2(sc[2 * e]);
            const float p1 = fast_exp2(sc[2 * e + 1]);
            dsk[e] = E::pack2(p0 * dp[2 * e], p1 * dp[2 * e + 1]);
          }
#pragma unroll
          for (int dc = 0; dc < G::DC; ++dc) {
#pragma unroll
            for (int kh = 0; kh < 2; ++kh) {
              const u32x4_t df = {dsk[4 * kh], dsk[4 * kh + 1], dsk[4 * kh + 2], dsk[4 * kh + 3]};
              acc[dc] = E::mfma(tr_frag(tK, kh, dc), df, acc[dc]);
            }
          }
        }
      }
    };
    if constexpr (kDma)
      run_groups_dma<NG, true>(nb, issue_dma, body);
    else
      run_groups<kLook, NG>(nb, issue_regs, put_regs, body);
  };
  if (exact)
    run(std::true_type{});
  else
    run(std::false_type{});

  uint16_t* orow = a.dq + b * a.sdq.b + h * a.sdq.h + (int64_t)qsafe * a.sdq.n;
  const float sc = a.sm_scale;
  auto piece = [&](int dc, int ii) {
    return u32x2_t{E::pack2(acc[dc][4 * ii] * sc, acc[dc][4 * ii + 1] * sc),
                   E::pack2(acc[dc][4 * ii + 2] * sc, acc[dc][4 * ii + 3] * sc)};
  };
  // Head dims of 64 and more with 16-byte aligned rows: dQ goes through the wave's idle LDS tile so
  // every global store writes whole rows.
  bool staged = false;
  if constexpr (D >= 64) {
    if (rows16_ok(a.dq, a.sdq)) {
      const int q0 = tp.tile * kTile + wave * kBlock;
      store_rows_via_lds<D>(wave_tile(sK, wave), lane, a.dq + b * a.sdq.b + h * a.sdq.h + (int64_t)q0 * a.sdq.n,
                            a.sdq.n, imin(kBlock, m.N - q0), piece);
      staged = true;
    }
  }
  if (qvalid && !staged) {
#pragma unroll
    for (int dc = 0; dc < G::DC; ++dc) {
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int d0 = 32 * dc + 8 * ii + 4 * g;
        if (d0 < D) *reinterpret_cast<u32x2_t*>(orow + d0) = piece(dc, ii);
      }
    }
  }
}

// Register-staged query chunk y of a dK/dV group (head dims below 64): Q and dO rows, plus (in wave
// y only) the chunk's -LSE (lanes 0-31) or -Delta (lanes 32-63) of query row lane % 32.
template <int D>
struct ChunkRegs {
  TileRegs<D> q, o;
  uint32_t seed;  // raw bits
};

template <int D, class E>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(bwd_waves<D>(), 8))) void attn_bwd_dkdv_kernel(const AttnArgs a) {
  using G = TileGeom<D>;
  constexpr int NG = bwd_group<D>();
  // Head dims of 64 and more stage Q / dO chunks and their seeds by direct global -> LDS loads into
  // dense swizzled tiles; smaller ones through registers into padded tiles.
  constexpr bool kDma = D >= 64;
  using DT = DmaTile<kDma ? D : 64, D != 256>;  // D = 256: the register-lean swizzle (fewer spills)
  constexpr bool kSkew = D == 64 && NG == 4;
  constexpr int kSkewMaxChunks = 16;
  constexpr int TE = kDma ? DT::ELEMS : G::ELEMS;
  __shared__ __attribute__((aligned(16))) uint16_t sQ[2][NG][TE];  // [buffer][chunk of the group]
  __shared__ __attribute__((aligned(16))) uint16_t sDO[2][NG][TE];
  // -LSE of the chunk's query rows in [0, kBlock), their -Delta in [kBlock, 2 kBlock).
  __shared__ __attribute__((aligned(16))) float sSeed[2][NG][2 * kBlock];
  __shared__ int s_span[2 * kWaves];
  __shared__ int s_steps[kWaves];

  const MaskSpec m = a.m;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_index<D>();
  const int g = lane >> 5, c32 = lane & 31;
  int b, h;
  TilePlan tp;
  k_workgroup(a, b, h, tp);
  const RowView row = row_view(a, b, tp.mono);
  KState st;
  int run_end;
  // (The f16 dK/dV kernel at D = 256 keeps the span reductions: with the four-lane reads the
  // compiler's AGPR-copy rewrite crashes on it.)
  constexpr bool kMono = D != 256;
  const bool planned = k_begin<kMono>(a, tp, row, s_span, st, run_end);
  const int kp = st.kp;
  const bool kvalid = st.kvalid;
  const int nc = st.nc;
  const bool exact = row.mono;
  const int64_t dk_doc = (!exact && kvalid) ? load_doc(a, b, kp) : 0;
  // Skewed schedule: wave w's keys start 2w chunks after the tile's first key, and a temporary-stream
  // key with a short window sees only a few chunks, so waves sharing one 4-chunk group would each be
  // busy in about half of it. Instead, at step s wave w takes chunk 2w + s: the eight staged chunks
  // (both buffers, as one ring of slots) always hold chunks s .. s + 7, every wave has a block at
  // each step, and one chunk enters the ring per step.
  const bool skew = kSkew && st.stream == STREAM_TEMPORARY && nc > 0 && nc <= kSkewMaxChunks &&
                    (stream_pos(m, st.stream, st.first) >> 5) == st.c0;

  const BufRsrc q_src = head_rsrc<D>(a.q + b * a.sq.b + h * a.sq.h, a.sq.n, m.N);
  const BufRsrc o_src = head_rsrc<D>(a.dO + b * a.sdo.b + h * a.sdo.h, a.sdo.n, m.N);
  // Seeds of this (row, head): -LSE of every query, then -Delta of every query (written by the dQ pass).
  const BufRsrc seed_src = make_rsrc(a.seeds + ((int64_t)b * a.H + h) * 2 * m.N, (uint32_t)(2 * m.N * 4));

  // K and V fragments: B operands of S = Q K^T and dP = dO V^T (lane: key c32, d = 16c + 8g ..).
  u32x4_t kf[D / 16], vf[D / 16];
  {
    const uint16_t* krow = a.k + b * a.sk.b + h * a.sk.h + (int64_t)kp * a.sk.n;
    const uint16_t* vrow = a.v + b * a.sv.b + h * a.sv.h + (int64_t)kp * a.sv.n;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      u32x4_t z = {0u, 0u, 0u, 0u};
      kf[c] = kvalid ? *reinterpret_cast<const u32x4_t*>(krow + 16 * c + 8 * g) : z;
      vf[c] = kvalid ? *reinterpret_cast<const u32x4_t*>(vrow + 16 * c + 8 * g) : z;
    }
  }
  if constexpr (!kDma) {
#pragma unroll
    for (int x = 0; x < 2; ++x) {
#pragma unroll
      for (int y = 0; y < NG; ++y) {
        zero_pad_cols<D>(sQ[x][y], tid);
        zero_pad_cols<D>(sDO[x][y], tid);
      }
    }
  }

  // Byte offset of chunk i's first row: i * (bytes per chunk) + the first chunk's offset.
  const uint32_t q_blk = (uint32_t)(kBlock * a.sq.n * 2), o_blk = (uint32_t)(kBlock * a.sdo.n * 2);
  const uint32_t q_c0 = (uint32_t)((int64_t)st.c0 * kBlock * a.sq.n * 2);
  const uint32_t o_c0 = (uint32_t)((int64_t)st.c0 * kBlock * a.sdo.n * 2);
  // Byte offset, within the seed buffer, of the seed lane `lane` stages for chunk i (wave y of the
  // group stages chunk y's): -LSE for lanes 0-31, -Delta for lanes 32-63, of query row lane % 32.
  auto seed_off = [&](int i) {
    return (uint32_t)(((lane >> 5) * m.N + imin((st.c0 + i) * kBlock + c32, m.N - 1)) * 4);
  };

  // Register staging (head dims below 64).
  ChunkRegs<D> rc[kLook][NG];
  const auto q_off = TileRegs<D>::offsets(tid, (uint32_t)(a.sq.n * 2));
  const auto o_off = TileRegs<D>::offsets(tid, (uint32_t)(a.sdo.n * 2));
  auto issue_regs = [&](int j, int slot) {
#pragma unroll
    for (int y = 0; y < NG; ++y) {
      const int i = NG * j + y;
      if (i < nc) {
        rc[slot][y].q.load(q_src, q_c0 + (uint32_t)i * q_blk, q_off, tid);
        rc[slot][y].o.load(o_src, o_c0 + (uint32_t)i * o_blk, o_off, tid);
        if (wave == y % kWaves) rc[slot][y].seed = __builtin_amdgcn_raw_buffer_load_b32(seed_src, seed_off(i), 0, 0);
      }
    }
  };
  auto put_regs = [&](int slot, int buf) {
#pragma unroll
    for (int y = 0; y < NG; ++y) {
      rc[slot][y].q.store(sQ[buf][y], tid);
      rc[slot][y].o.store(sDO[buf][y], tid);
      if (wave == y % kWaves) sSeed[buf][y][lane] = __builtin_bit_cast(float, rc[slot][y].seed);
    }
  };
  // LDS-DMA staging (head dims of 64 and more).
  const auto q_dma = DT::sources(tid, (uint32_t)(a.sq.n * 2));
  const auto o_dma = DT::sources(tid, (uint32_t)(a.sdo.n * 2));
  auto issue_dma = [&](int j, int buf) {
#pragma unroll
    for (int y = 0; y < NG; ++y) {
      const int i = NG * j + y;
      if (i < nc) {
        DT::load(q_src, q_c0 + (uint32_t)i * q_blk, q_dma, sQ[buf][y], wave);
        DT::load(o_src, o_c0 + (uint32_t)i * o_blk, o_dma, sDO[buf][y], wave);
        if (wave == y % kWaves) lds_dma_b32(seed_src, sSeed[buf][y], seed_off(i));
      }
    }
  };
  // Fragment reads of a staged chunk tile.
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

  f32x16_t dk[G::DC], dv[G::DC];
#pragma unroll
  for (int dc = 0; dc < G::DC; ++dc) {
    dk[dc] = f32x16_t{};
    dv[dc] = f32x16_t{};
  }

  auto run = [&](auto exact_tag) {
    constexpr bool EXACT = decltype(exact_tag)::value;
    // The first group's loads go out with the lanes' run ends and the K/V fragments; what depends
    // on those waits below, for all of them at once.
    if constexpr (kDma)
      issue_dma(0, 0);
    else
      issue_regs(0, 0);
    if constexpr (kSkew)
      if (skew) issue_dma(1, 1);
    if (planned) k_lanes<kMono>(m, run_end, st);
    // The dP tile starts from the -Delta seeds of its query rows, so it comes out of the MFMAs as
    // dP - Delta and dS = P * dP' is one VALU operation per element; the S tile is scaled in fp32 by
    // one FMA per score with the -LSE seeds (S * scale2 - LSE), never by rounding a scaled K.
    const float scale2 = a.scale2;
    auto cls_of = [&](int i) { return classify_block(st.w, (st.c0 + i) * kBlock, EXACT); };
    const BlockMask bm = k_block_mask(st, EXACT);
    // S and dP tiles of block y of the group (the dP tile starts from its rows' -Delta seeds).
    auto sdp = [&](const uint16_t* tQ, const uint16_t* tDO, const float* seed, f32x16_t& sc, f32x16_t& dp) {
      sc = f32x16_t{};
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        // Query rows 8*i4 + 4g + {0..3} of this chunk.
        const f32x4_t d4 = *reinterpret_cast<const SPS_LDS f32x4_t*>(
            (const SPS_LDS float*)(seed + kBlock + 8 * i4 + 4 * g));
#pragma unroll
        for (int t = 0; t < 4; ++t) dp[4 * i4 + t] = d4[t];
      }
#pragma unroll
      for (int c = 0; c < D / 16; ++c) {
        sc = E::mfma(row_frag(tQ, c), kf[c], sc);
        dp = E::mfma(row_frag(tDO, c), vf[c], dp);
      }
    };
    // Block y's S tile in fp32 (S * scale2 - LSE, the -LSE seeds read here), masked when partial.
    auto scores = [&](const float* seed, int qc, bool full, f32x16_t& sc) {
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const f32x4_t l4 = *reinterpret_cast<const SPS_LDS f32x4_t*>(
            (const SPS_LDS float*)(seed + 8 * i4 + 4 * g));
#pragma unroll
        for (int t = 0; t < 4; ++t) sc[4 * i4 + t] = __builtin_fmaf(sc[4 * i4 + t], scale2, l4[t]);
      }
      if (!full)
        mask_partial<EXACT>(sc, st.r, st.w, qc, g, [&] { return ks_exact_bits(a, b, kp, st.r.hi, qc, g, dk_doc); });
    };
    // P and dS of block y, then the dV and dK products.
    auto grads = [&](const uint16_t* tQ, const uint16_t* tDO, const f32x16_t& sc, const f32x16_t& dp) {
      uint32_t pk[8], dsk[8];
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        float p[4], ds[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int e = 4 * i4 + t;
          p[t] = fast_exp2(sc[e]);
          ds[t] = p[t] * dp[e];
        }
        pk[2 * i4] = E::pack2(p[0], p[1]);
        pk[2 * i4 + 1] = E::pack2(p[2], p[3]);
        dsk[2 * i4] = E::pack2(ds[0], ds[1]);
        dsk[2 * i4 + 1] = E::pack2(ds[2], ds[3]);
      }
#pragma unroll
      for (int dc = 0; dc < G::DC; ++dc) {
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
          const u32x4_t pf = {pk[4 * kh], pk[4 * kh + 1], pk[4 * kh + 2], pk[4 * kh + 3]};
          const u32x4_t df = {dsk[4 * kh], dsk[4 * kh + 1], dsk[4 * kh + 2], dsk[4 * kh + 3]};
          dv[dc] = E::mfma(tr_frag(tDO, kh, dc), pf, dv[dc]);
          dk[dc] = E::mfma(tr_frag(tQ, kh, dc), df, dk[dc]);
        }
      }
    };
    auto block = [&](const uint16_t* tQ, const uint16_t* tDO, const float* seed, int qc, bool full) {
      f32x16_t sc, dp;
      sdp(tQ, tDO, seed, sc, dp);
      scores(seed, qc, full, sc);
      grads(tQ, tDO, sc, dp);
    };
    auto body = [&](int j, int buf) {
      int act2, full2;
      group_codes<NG>(bm, NG * j, nc, cls_of, act2, full2);
#pragma unroll
      for (int y = 0; y < NG; ++y) {
        if ((act2 >> y) & 1) block(sQ[buf][y], sDO[buf][y], sSeed[buf][y], (st.c0 + NG * j + y) * kBlock, (full2 >> y) & 1);
      }
    };
    if constexpr (kSkew) {
      if (skew) {
        // Chunk c sits in slot c % 8 = (buffer, chunk of the group) (c % 8 / 4, c % 4). Chunks 0-7
        // were loaded by direct LDS loads before the lanes' setup; chunk s + 8 goes through
        // registers during step s and is written at the start of step s + 1 into the slot of chunk
        // s, which every wave has finished with by then (its last reader, wave 0, took it at step s).
        uint16_t* const ringQ = &sQ[0][0][0];
        uint16_t* const ringO = &sDO[0][0][0];
        float* const ringS = &sSeed[0][0][0];
        const uint64_t act = bm.act0, full = bm.full0;  // nc <= 16: every chunk's bit is in word 0
        // Steps: until every wave has reached its last active chunk.
        if (lane == 0) s_steps[wave] = (act ? 63 - __builtin_clzll(act) : -1) - 2 * wave + 1;
        vmem_wait_all();
        __syncthreads();
        int steps = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) steps = imax(steps, s_steps[w]);
        steps = wave_uniform(steps);
        u32x4_t rq = {0u, 0u, 0u, 0u}, ro = {0u, 0u, 0u, 0u};
        uint32_t rs = 0u;
        for (int sp = 0; sp < steps; ++sp) {
          if (sp > 0) {
            const int c = sp + 7;
            if (c < nc) {
              const int sl = c & 7;
              lds_write_b128(ringQ + sl * TE + tid * 8, rq);
              lds_write_b128(ringO + sl * TE + tid * 8, ro);
              if (wave == (c & 3)) ringS[sl * 2 * kBlock + lane] = __builtin_bit_cast(float, rs);
            }
          }
          {
            const int c = sp + 8;
            if (c < nc) {
              rq = buf_load_b128(q_src, q_c0 + (uint32_t)c * q_blk + q_dma.o[0]);
              ro = buf_load_b128(o_src, o_c0 + (uint32_t)c * o_blk + o_dma.o[0]);
              if (wave == (c & 3)) rs = __builtin_amdgcn_raw_buffer_load_b32(seed_src, seed_off(c), 0, 0);
            }
          }
          const int i = 2 * wave + sp;
          if (i < nc && ((act >> i) & 1ull)) {
            const int sl = i & 7;
            block(ringQ + sl * TE, ringO + sl * TE, ringS + sl * 2 * kBlock, (st.c0 + i) * kBlock, (full >> i) & 1ull);
          }
          lds_barrier();
        }
        return;
      }
    }
    if constexpr (kDma)
      run_groups_dma<NG, true>(nc, issue_dma, body);
    else
      run_groups<kLook, NG, true>(nc, issue_regs, put_regs, body);
  };
  if (exact)
    run(std::true_type{});
  else
    run(std::false_type{});

  const float sc = a.sm_scale;
  // Pieces of the lane's key row: d = 32 dc + 8 ii + 4 g .. +3 of dK (scaled by sm_scale) and dV.
  auto piece_k = [&](int dc, int ii) {
    return u32x2_t{E::pack2(dk[dc][4 * ii] * sc, dk[dc][4 * ii + 1] * sc),
                   E::pack2(dk[dc][4 * ii + 2] * sc, dk[dc][4 * ii + 3] * sc)};
  };
  auto piece_v = [&](int dc, int ii) {
    return u32x2_t{E::pack2(dv[dc][4 * ii], dv[dc][4 * ii + 1]), E::pack2(dv[dc][4 * ii + 2], dv[dc][4 * ii + 3])};
  };
  // With dense tiles and 16-byte aligned output rows the wave's 32 rows go through its own part of
  // the (now idle) first staging buffer, so every global store writes whole rows (dK/dV -4.6 % at C3).
  bool staged = false;
  if constexpr (kDma) {
    if (rows16_ok(a.dk, a.sdk) && rows16_ok(a.dv, a.sdv)) {
      // The wave's keys are consecutive indices of one stream: rows `step` positions apart.
      const int t0 = st.first + wave * kBlock;
      const int p0 = stream_pos(m, st.stream, t0);
      const int nrows = imin(kBlock, stream_len(m.family, m.N, st.stream, m.P) - t0);
      const int kstep = m.family == FAMILY_FULL ? 1 : 2;
      store_rows_via_lds<D>(wave_tile(sQ, wave), lane, a.dk + b * a.sdk.b + h * a.sdk.h + (int64_t)p0 * a.sdk.n,
                            kstep * a.sdk.n, nrows, piece_k);
      store_rows_via_lds<D>(wave_tile(sDO, wave), lane, a.dv + b * a.sdv.b + h * a.sdv.h + (int64_t)p0 * a.sdv.n,
                            kstep * a.sdv.n, nrows, piece_v);
      staged = true;
    }
  }
  if (!staged && kvalid) {
    uint16_t* dkrow = a.dk + b * a.sdk.b + h * a.sdk.h + (int64_t)kp * a.sdk.n;
    uint16_t* dvrow = a.dv + b * a.sdv.b + h * a.sdv.h + (int64_t)kp * a.sdv.n;
#pragma unroll
    for (int dc = 0; dc < G::DC; ++dc) {
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int d0 = 32 * dc + 8 * ii + 4 * g;
        if (d0 < D) {
          *reinterpret_cast<u32x2_t*>(dkrow + d0) = piece_k(dc, ii);
          *reinterpret_cast<u32x2_t*>(dvrow + d0) = piece_v(dc, ii);
        }
      }
    }
  }
}

// Writes the visibility mask exactly as the key-stationary dK/dV kernel evaluates it.
__global__ __launch_bounds__(256) void mask_dump_kv_kernel(const AttnArgs a) {
  __shared__ int s_span[2 * kWaves];
  const MaskSpec m = a.m;
  const int tid = threadIdx.x, lane = tid & 63;
  const int g = lane >> 5;
  int b, h;
  TilePlan tp;
  k_workgroup(a, b, h, tp);
  const RowView row = row_view(a, b, tp.mono);
  KState st;
  int run_end;
  if (k_begin(a, tp, row, s_span, st, run_end)) k_lanes(m, run_end, st);
  const bool exact = row.mono;
  const int64_t dk_doc = (!exact && st.kvalid) ? load_doc(a, b, st.kp) : 0;
  const BlockMask bm = k_block_mask(st, exact);
  for (int i = 0; i < st.nc; ++i) {
    const int qc = (st.c0 + i) * kBlock;
    const int cls = i < 128 ? mask_class(bm, i) : classify_block(st.w, qc, exact);
    if (cls == TILE_SKIP || !st.kvalid) continue;
    uint32_t bits = 0xffffu;
    if (cls == TILE_PARTIAL) {
      f32x16_t z = {};
      auto exact_bits = [&] { return ks_exact_bits(a, b, st.kp, st.r.hi, qc, g, dk_doc); };
      if (exact)
        mask_partial<true>(z, st.r, st.w, qc, g, exact_bits);
      else
        mask_partial<false>(z, st.r, st.w, qc, g, exact_bits);
      bits = 0;
      for (int e = 0; e < 16; ++e) bits |= (uint32_t)(z[e] == 0.f) << e;
    }
    for (int e = 0; e < 16; ++e) {
      const int qp = qc + acc_row(e, g);
      if (((bits >> e) & 1u) && qp < m.N) a.mask_out[((int64_t)b * m.N + qp) * m.N + st.kp] = 1;
    }
  }
}

template <int D, class E>
static hipError_t launch_bwd_t(const AttnArgs& a, int passes, hipStream_t stream) {
  const int64_t nq = (int64_t)q_tiles(a.m.N) * a.B * a.H;
  const int64_t nk = (int64_t)k_tiles(a.m.family, a.m.N, a.m.P) * a.B * a.H;
  if ((passes & kBwdDq) && nq > 0) {
    hipLaunchKernelGGL((attn_bwd_dq_kernel<D, E>), dim3((unsigned)nq), dim3(256), 0, stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if ((passes & kBwdDkdv) && nk > 0) {
    hipLaunchKernelGGL((attn_bwd_dkdv_kernel<D, E>), dim3((unsigned)nk), dim3(256), 0, stream, a);
    return hipGetLastError();
  }
  return hipSuccess;
}

hipError_t launch_attn_bwd(const AttnArgs& a, int D, int is_f16, int passes, hipStream_t stream) {
#define SPS_BWD_CASE(DD)                                                                                  \
  case DD:                                                                                                \
    return is_f16 ? launch_bwd_t<DD, ElemF16>(a, passes, stream) : launch_bwd_t<DD, ElemBF16>(a, passes, stream);
  switch (D) {
    SPS_BWD_CASE(16)
    SPS_BWD_CASE(32)
    SPS_BWD_CASE(64)
    SPS_BWD_CASE(128)
    SPS_BWD_CASE(256)
    default:
      return hipErrorInvalidValue;
  }
#undef SPS_BWD_CASE
}

hipError_t launch_mask_dump_q(const AttnArgs& a, hipStream_t stream);

hipError_t launch_mask_dump(const AttnArgs& a, int schedule, hipStream_t stream) {
  if (schedule == 0) return launch_mask_dump_q(a, stream);
  const int n = k_tiles(a.m.family, a.m.N, a.m.P) * a.B * a.H;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(mask_dump_kv_kernel, dim3(n), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace sps
