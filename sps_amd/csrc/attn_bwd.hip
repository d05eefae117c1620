// Backward attention, bf16/f16 MFMA, gfx950. Two deterministic passes, no atomics, as in the
// reference (_sps_bwd_dq_kernel / _sps_bwd_dkdv_kernel, triton_sps_flash_attention.py:272-488;
// reverse twins triton_reverse_sps_flash_attention.py:370-599; full triton_full_flash_attention.py:301-460):
//
//  1. dQ pass (query-stationary, the forward's block schedule). Its prologue computes
//     Delta = rowsum(O * dO) for its own queries and stores it for pass 2 (this replaces the
//     reference's separate _attn_bwd_preprocess launch). Per 32-key block:
//       S^T = K Q^T, dP^T = V dO^T (K, V rows from LDS; Q, dO in registers),
//       P = exp2(S*scale2 - LSE), dS = P (dP - Delta)   (lane-local LSE and Delta),
//       dQ^T += K^T dS^T  (K^T fragments via ds_read_b64_tr_b16).
//  2. dK/dV pass (key-stationary). A workgroup owns 128 keys of one stream (natural, persistent
//     or temporary), each wave 32 of them held in registers; it walks 32-query chunks that can see
//     those keys (persistent keys: diagonal to document end; temporary keys: the w-token window):
//       S = Q K^T, dP = dO V^T (Q, dO rows from LDS; K, V in registers),
//       dV^T += dO^T P, dK^T += Q^T dS (dO^T, Q^T fragments via ds_read_b64_tr_b16).
// dK and dQ are scaled by sm_scale at the end, as in the reference.
#include "attn_tiles.hpp"

namespace sps {

template <int D, class E>
__global__ __launch_bounds__(256) void attn_bwd_dq_kernel(const AttnArgs a) {
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
  const int qt = nqt - 1 - (lid - bh * nqt);
  const int b = bh / a.H, h = bh - b * a.H;
  const int qa = qt * kTile;
  const int qw = qa + wave * kBlock;
  const int qp = qw + c32;
  const bool qvalid = qp < m.N;
  const int qsafe = qvalid ? qp : 0;

  const uint16_t* kbase = a.k + b * a.sk.b + h * a.sk.h;
  const uint16_t* vbase = a.v + b * a.sv.b + h * a.sv.h;
  const int64_t* gmin = a.gmin + (int64_t)b * a.NG;
  const int64_t* gmax = a.gmax + (int64_t)b * a.NG;

  // Q and dO fragments (B operands; lane: query c32, d = 16c + 8g .. +7) and Delta.
  u32x4_t qf[D / 16], dof[D / 16];
  float delta;
  {
    const uint16_t* qrow = a.q + b * a.sq.b + h * a.sq.h + (int64_t)qsafe * a.sq.n;
    const uint16_t* dorow = a.dO + b * a.sdo.b + h * a.sdo.h + (int64_t)qsafe * a.sdo.n;
    const uint16_t* orow = a.o + b * a.so.b + h * a.so.h + (int64_t)qsafe * a.so.n;
    float part = 0.f;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      u32x4_t z = {0u, 0u, 0u, 0u};
      qf[c] = qvalid ? *reinterpret_cast<const u32x4_t*>(qrow + 16 * c + 8 * g) : z;
      dof[c] = qvalid ? *reinterpret_cast<const u32x4_t*>(dorow + 16 * c + 8 * g) : z;
      const u32x4_t of = qvalid ? *reinterpret_cast<const u32x4_t*>(orow + 16 * c + 8 * g) : z;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        part += E::to_f32((uint16_t)(of[j] & 0xffffu)) * E::to_f32((uint16_t)(dof[c][j] & 0xffffu));
        part += E::to_f32((uint16_t)(of[j] >> 16)) * E::to_f32((uint16_t)(dof[c][j] >> 16));
      }
    }
    delta = half_sum(part);
  }
  const int64_t rowid = (int64_t)bh * m.N + qsafe;
  if (qvalid && g == 0) a.delta[rowid] = delta;
  const float lse = qvalid ? a.lse[rowid] : 0.f;
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
      f32x16_t sc = {}, dp = {};
#pragma unroll
      for (int c = 0; c < D / 16; ++c) {
        sc = E::mfma(lds_read_b128(tK + c32 * G::RS + 16 * c + 8 * g), qf[c], sc);
        dp = E::mfma(lds_read_b128(tV + c32 * G::RS + 16 * c + 8 * g), dof[c], dp);
      }
      const uint32_t bits = cls == TILE_PARTIAL ? qs_mask_bits(m, qp, dq, kr_cur, g, sDoc[buf]) : 0xffffu;
      uint32_t dsk[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float p0 = fast_exp2(fmaf(sc[2 * j], a.scale2, -lse));
        float p1 = fast_exp2(fmaf(sc[2 * j + 1], a.scale2, -lse));
        p0 = ((bits >> (2 * j)) & 1u) ? p0 : 0.f;
        p1 = ((bits >> (2 * j + 1)) & 1u) ? p1 : 0.f;
        dsk[j] = E::pack2(p0 * (dp[2 * j] - delta), p1 * (dp[2 * j + 1] - delta));
      }
#pragma unroll
      for (int dc = 0; dc < G::DC; ++dc) {
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
          const u32x4_t df = {dsk[4 * kh], dsk[4 * kh + 1], dsk[4 * kh + 2], dsk[4 * kh + 3]};
          acc[dc] = E::mfma(lds_frag_tr(tK, G::RS, 16 * kh, 32 * dc, lane), df, acc[dc]);
        }
      }
    }

    if (nxt < nb) store_block(buf ^ 1);
    __syncthreads();
    buf ^= 1;
    cur = nxt;
    kr_cur = kr_nxt;
  }

  if (qvalid) {
    uint16_t* row = a.dq + b * a.sdq.b + h * a.sdq.h + (int64_t)qp * a.sdq.n;
    const float sc = a.sm_scale;
#pragma unroll
    for (int dc = 0; dc < G::DC; ++dc) {
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int d0 = 32 * dc + 8 * ii + 4 * g;
        if (d0 < D) {
          u32x2_t w = {E::pack2(acc[dc][4 * ii] * sc, acc[dc][4 * ii + 1] * sc),
                       E::pack2(acc[dc][4 * ii + 2] * sc, acc[dc][4 * ii + 3] * sc)};
          *reinterpret_cast<u32x2_t*>(row + d0) = w;
        }
      }
    }
  }
}

template <int D, class E>
__global__ __launch_bounds__(256) void attn_bwd_dkdv_kernel(const AttnArgs a) {
  using G = TileGeom<D>;
  __shared__ __attribute__((aligned(16))) uint16_t sQ[2][G::ELEMS];
  __shared__ __attribute__((aligned(16))) uint16_t sDO[2][G::ELEMS];
  __shared__ __attribute__((aligned(16))) float sLse[2][kBlock];
  __shared__ __attribute__((aligned(16))) float sDelta[2][kBlock];
  __shared__ int64_t sDoc[2][kBlock];

  const MaskSpec m = a.m;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, c32 = lane & 31;

  const int nkt = ktiles_per_head(m.family, m.N);
  const int lid = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = lid / nkt;
  const int kt = lid - bh * nkt;
  const int b = bh / a.H, h = bh - b * a.H;
  const KeyRun wg_run = ktile_run(m.family, m.N, kt);
  KeyRun w_run = wg_run;
  w_run.count = kBlock;
  w_run.first = wg_run.first + wave * kBlock;
  const int kp = key_pos(m, w_run, c32);
  const bool kvalid = kp < m.N;
  const int ksafe = kvalid ? kp : 0;

  const int64_t* gmin = a.gmin + (int64_t)b * a.NG;
  const int64_t* gmax = a.gmax + (int64_t)b * a.NG;
  const uint16_t* qbase = a.q + b * a.sq.b + h * a.sq.h;
  const uint16_t* dobase = a.dO + b * a.sdo.b + h * a.sdo.h;
  const float* lse_row = a.lse + (int64_t)bh * m.N;
  const float* delta_row = a.delta + (int64_t)bh * m.N;

  // K and V fragments: B operands of S = Q K^T and dP = dO V^T (lane: key c32, d = 16c + 8g ..).
  u32x4_t kf[D / 16], vf[D / 16];
  {
    const uint16_t* krow = a.k + b * a.sk.b + h * a.sk.h + (int64_t)ksafe * a.sk.n;
    const uint16_t* vrow = a.v + b * a.sv.b + h * a.sv.h + (int64_t)ksafe * a.sv.n;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      u32x4_t z = {0u, 0u, 0u, 0u};
      kf[c] = kvalid ? *reinterpret_cast<const u32x4_t*>(krow + 16 * c + 8 * g) : z;
      vf[c] = kvalid ? *reinterpret_cast<const u32x4_t*>(vrow + 16 * c + 8 * g) : z;
    }
  }
  const int64_t dk_doc = (m.has_docs && kvalid) ? load_doc(a, b, kp) : 0;

  const KSchedule s = make_kschedule(m, wg_run);
  const int ce = s.c0 + s.nc;
  DocRange wg_kd = run_docs(m, wg_run, gmin, gmax);
  DocRange w_kd = run_docs(m, w_run, gmin, gmax);

  zero_pad_cols<D>(sQ[0], tid);
  zero_pad_cols<D>(sQ[1], tid);
  zero_pad_cols<D>(sDO[0], tid);
  zero_pad_cols<D>(sDO[1], tid);

  TileRegs<D> rq, rdo;
  float rl = 0.f, rd = 0.f;
  int64_t rdoc = 0;
  auto load_chunk = [&](int c) {
    const int q0 = c * kBlock;
    auto pos = [&](int r) { return q0 + r; };
    rq.load(qbase, a.sq.n, m.N, tid, pos);
    rdo.load(dobase, a.sdo.n, m.N, tid, pos);
    if (tid < kBlock) {
      const int qp = q0 + tid;
      const bool ok = qp < m.N;
      rl = ok ? lse_row[qp] : 0.f;
      rd = ok ? delta_row[qp] : 0.f;
      rdoc = (m.has_docs && ok) ? load_doc(a, b, qp) : INT64_MIN;
    }
  };
  auto store_chunk = [&](int buf) {
    rq.store(sQ[buf], tid);
    rdo.store(sDO[buf], tid);
    if (tid < kBlock) {
      sLse[buf][tid] = rl;
      sDelta[buf][tid] = rd;
      sDoc[buf][tid] = rdoc;
    }
  };

  f32x16_t dk[G::DC], dv[G::DC];
#pragma unroll
  for (int dc = 0; dc < G::DC; ++dc) {
    dk[dc] = f32x16_t{};
    dv[dc] = f32x16_t{};
  }

  int cur = ks_next_chunk(m, s, wg_run, wg_kd, gmin, gmax, s.c0 - 1);
  if (cur < ce) {
    load_chunk(cur);
    store_chunk(0);
  }
  __syncthreads();
  int buf = 0;
  while (cur < ce) {
    const int nxt = ks_next_chunk(m, s, wg_run, wg_kd, gmin, gmax, cur);
    if (nxt < ce) load_chunk(nxt);

    const int qc = cur * kBlock;
    const int qhi = qc + kBlock - 1 < m.N - 1 ? qc + kBlock - 1 : m.N - 1;
    DocRange qd = {0, 0};
    if (m.has_docs) qd = doc_range(gmin, gmax, qc, qhi);
    const int cls = classify(m, qc, qhi, w_run, qd, w_kd);
    if (cls != TILE_SKIP) {
      const uint16_t* tQ = sQ[buf];
      const uint16_t* tDO = sDO[buf];
      f32x16_t sc = {}, dp = {};
#pragma unroll
      for (int c = 0; c < D / 16; ++c) {
        sc = E::mfma(lds_read_b128(tQ + c32 * G::RS + 16 * c + 8 * g), kf[c], sc);
        dp = E::mfma(lds_read_b128(tDO + c32 * G::RS + 16 * c + 8 * g), vf[c], dp);
      }
      const uint32_t bits = cls == TILE_PARTIAL ? ks_mask_bits(m, qc, kp, dk_doc, g, sDoc[buf]) : 0xffffu;
      uint32_t pk[8], dsk[8];
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        // Query rows 8*i4 + 4g + {0..3} of this chunk.
        const f32x4_t l4 = *reinterpret_cast<const SPS_LDS f32x4_t*>(
            (const SPS_LDS float*)(&sLse[buf][8 * i4 + 4 * g]));
        const f32x4_t d4 = *reinterpret_cast<const SPS_LDS f32x4_t*>(
            (const SPS_LDS float*)(&sDelta[buf][8 * i4 + 4 * g]));
        float p[4], ds[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int i = 4 * i4 + t;
          float pv = fast_exp2(fmaf(sc[i], a.scale2, -l4[t]));
          pv = ((bits >> i) & 1u) ? pv : 0.f;
          p[t] = pv;
          ds[t] = pv * (dp[i] - d4[t]);
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
          dv[dc] = E::mfma(lds_frag_tr(tDO, G::RS, 16 * kh, 32 * dc, lane), pf, dv[dc]);
          dk[dc] = E::mfma(lds_frag_tr(tQ, G::RS, 16 * kh, 32 * dc, lane), df, dk[dc]);
        }
      }
    }

    if (nxt < ce) store_chunk(buf ^ 1);
    __syncthreads();
    buf ^= 1;
    cur = nxt;
  }

  if (kvalid) {
    uint16_t* dkrow = a.dk + b * a.sdk.b + h * a.sdk.h + (int64_t)kp * a.sdk.n;
    uint16_t* dvrow = a.dv + b * a.sdv.b + h * a.sdv.h + (int64_t)kp * a.sdv.n;
    const float sc = a.sm_scale;
#pragma unroll
    for (int dc = 0; dc < G::DC; ++dc) {
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int d0 = 32 * dc + 8 * ii + 4 * g;
        if (d0 < D) {
          u32x2_t wk = {E::pack2(dk[dc][4 * ii] * sc, dk[dc][4 * ii + 1] * sc),
                        E::pack2(dk[dc][4 * ii + 2] * sc, dk[dc][4 * ii + 3] * sc)};
          u32x2_t wv = {E::pack2(dv[dc][4 * ii], dv[dc][4 * ii + 1]),
                        E::pack2(dv[dc][4 * ii + 2], dv[dc][4 * ii + 3])};
          *reinterpret_cast<u32x2_t*>(dkrow + d0) = wk;
          *reinterpret_cast<u32x2_t*>(dvrow + d0) = wv;
        }
      }
    }
  }
}

// Writes the visibility mask exactly as the key-stationary dK/dV kernel evaluates it.
__global__ __launch_bounds__(256) void mask_dump_kv_kernel(const AttnArgs a) {
  __shared__ int64_t sDoc[kBlock];
  const MaskSpec m = a.m;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, c32 = lane & 31;
  const int nkt = ktiles_per_head(m.family, m.N);
  const int b = blockIdx.x / nkt;
  const int kt = blockIdx.x - b * nkt;
  const KeyRun wg_run = ktile_run(m.family, m.N, kt);
  KeyRun w_run = wg_run;
  w_run.count = kBlock;
  w_run.first = wg_run.first + wave * kBlock;
  const int kp = key_pos(m, w_run, c32);
  const bool kvalid = kp < m.N;
  const int64_t* gmin = a.gmin + (int64_t)b * a.NG;
  const int64_t* gmax = a.gmax + (int64_t)b * a.NG;
  const int64_t dk_doc = (m.has_docs && kvalid) ? load_doc(a, b, kp) : 0;
  const KSchedule s = make_kschedule(m, wg_run);
  const int ce = s.c0 + s.nc;
  const DocRange wg_kd = run_docs(m, wg_run, gmin, gmax);
  const DocRange w_kd = run_docs(m, w_run, gmin, gmax);
  for (int cur = ks_next_chunk(m, s, wg_run, wg_kd, gmin, gmax, s.c0 - 1); cur < ce;
       cur = ks_next_chunk(m, s, wg_run, wg_kd, gmin, gmax, cur)) {
    const int qc = cur * kBlock;
    if (tid < kBlock) {
      const int qp = qc + tid;
      sDoc[tid] = (m.has_docs && qp < m.N) ? load_doc(a, b, qp) : INT64_MIN;
    }
    __syncthreads();
    const int qhi = qc + kBlock - 1 < m.N - 1 ? qc + kBlock - 1 : m.N - 1;
    DocRange qd = {0, 0};
    if (m.has_docs) qd = doc_range(gmin, gmax, qc, qhi);
    const int cls = classify(m, qc, qhi, w_run, qd, w_kd);
    if (cls != TILE_SKIP && kvalid) {
      const uint32_t bits = cls == TILE_FULL ? 0xffffu : ks_mask_bits(m, qc, kp, dk_doc, g, sDoc);
      for (int i = 0; i < 16; ++i) {
        const int qp = qc + acc_row(i, g);
        if (((bits >> i) & 1u) && qp < m.N) a.mask_out[((int64_t)b * m.N + qp) * m.N + kp] = 1;
      }
    }
    __syncthreads();
  }
}

template <int D, class E>
static hipError_t launch_bwd_t(const AttnArgs& a, int passes, hipStream_t stream) {
  const int nqt = (a.m.N + kTile - 1) / kTile;
  const int64_t nq = (int64_t)nqt * a.B * a.H;
  const int64_t nk = (int64_t)ktiles_per_head(a.m.family, a.m.N) * a.B * a.H;
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
    default:
      return hipErrorInvalidValue;
  }
#undef SPS_BWD_CASE
}

hipError_t launch_mask_dump_q(const AttnArgs& a, hipStream_t stream);

hipError_t launch_mask_dump(const AttnArgs& a, int schedule, hipStream_t stream) {
  if (schedule == 0) return launch_mask_dump_q(a, stream);
  const int n = ktiles_per_head(a.m.family, a.m.N) * a.B;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(mask_dump_kv_kernel, dim3(n), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace sps
