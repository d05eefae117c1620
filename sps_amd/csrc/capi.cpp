// C ABI of libsps_attn.so: argument validation, workspace layout and kernel dispatch.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/sps_attn.h"
#include "attn_kernels.hpp"
#include "decode_kernels.hpp"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return SPS_OK;
  return fail(SPS_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

constexpr size_t kAlign = 256;
size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The kernels read each (batch, head) slice through a 32-bit buffer descriptor, so the byte span of
// its N rows must stay below 2^31.
int check_tensor(const char* name, const void* p, const int64_t* st, int need, int N, int D) {
  if (!need) return SPS_OK;
  if (!p) return fail(SPS_E_INVALID, "%s: null pointer", name);
  if (!st) return fail(SPS_E_INVALID, "%s: null strides", name);
  if (!aligned16(p)) return fail(SPS_E_INVALID, "%s: base pointer must be 16-byte aligned", name);
  for (int i = 0; i < 3; ++i)
    if (st[i] % 8 != 0)
      return fail(SPS_E_INVALID, "%s: stride %d (%lld) must be a multiple of 8 elements", name, i,
                  (long long)st[i]);
  if (st[2] < 0) return fail(SPS_E_INVALID, "%s: negative sequence stride", name);
  if (((int64_t)N - 1) * st[2] * 2 + (int64_t)D * 2 > INT32_MAX)
    return fail(SPS_E_UNSUPPORTED, "%s: one head's rows span more than 2 GiB (N=%d, stride %lld)", name, N,
                (long long)st[2]);
  return SPS_OK;
}

sps::Strides3 strides(const int64_t* st) {
  sps::Strides3 s = {0, 0, 0};
  if (st) s = {st[0], st[1], st[2]};
  return s;
}

bool supported_head_dim(int D) { return D == 16 || D == 32 || D == 64 || D == 128 || D == 256; }

struct AttnLayout {
  size_t run_start, run_end, row_mono, q_plan, k_plan, seeds, total;
};

AttnLayout attn_layout(int family, int B, int H, int N, int has_docs, int backward) {
  AttnLayout l = {0, 0, 0, 0, 0, 0, 0};
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off = align_up(off + bytes);
    return at;
  };
  if (has_docs) {
    const int P = family == SPS_FAMILY_REVERSE_SPS ? 1 : 0;
    l.run_start = take((size_t)B * N * sizeof(int));
    l.run_end = take((size_t)B * N * sizeof(int));
    l.row_mono = take((size_t)B * sizeof(int));
    l.q_plan = take((size_t)B * sps::q_tiles(N) * sizeof(sps::TilePlan));
    l.k_plan = take((size_t)B * sps::k_tiles(family, N, P) * sizeof(sps::TilePlan));
  }
  if (backward) l.seeds = take((size_t)B * H * 2 * N * sizeof(float));
  l.total = off;
  return l;
}

// Fills the mask-related fields of the argument block and validates the common scalars.
int setup_common(sps::AttnArgs& a, int family, int B, int H, int N, const void* docs, int docs_dtype,
                 int64_t docs_stride_b, int window, int has_pkw, int pkw, void* workspace,
                 size_t workspace_bytes, int backward) {
  if (family < SPS_FAMILY_FULL || family > SPS_FAMILY_REVERSE_SPS)
    return fail(SPS_E_INVALID, "unknown attention family %d", family);
  if (B < 0 || H < 0 || N < 0) return fail(SPS_E_INVALID, "negative size B=%d H=%d N=%d", B, H, N);
  if (family != SPS_FAMILY_FULL && (N % 2) != 0)
    return fail(SPS_E_INVALID, "SPS families need an even sequence length (2T), got N=%d", N);
  if (N > (1 << 28)) return fail(SPS_E_UNSUPPORTED, "sequence length %d too large", N);
  if (docs && docs_dtype != SPS_DTYPE_I32 && docs_dtype != SPS_DTYPE_I64)
    return fail(SPS_E_INVALID, "document ids must be int32 or int64 (dtype code %d)", docs_dtype);
  const AttnLayout l = attn_layout(family, B, H, N, docs != nullptr, backward);
  if (workspace_bytes < l.total)
    return fail(SPS_E_WORKSPACE, "workspace too small: %zu bytes < %zu", workspace_bytes, l.total);
  if (l.total > 0 && !workspace) return fail(SPS_E_INVALID, "workspace: null pointer");
  char* ws = static_cast<char*>(workspace);
  std::memset(&a, 0, sizeof(a));
  a.docs = docs;
  a.docs_i64 = docs_dtype == SPS_DTYPE_I64;
  a.docs_sb = docs_stride_b;
  if (docs) {
    a.run_start = reinterpret_cast<int*>(ws + l.run_start);
    a.run_end = reinterpret_cast<int*>(ws + l.run_end);
    a.row_mono = reinterpret_cast<int*>(ws + l.row_mono);
    a.q_plan = reinterpret_cast<sps::TilePlan*>(ws + l.q_plan);
    a.k_plan = reinterpret_cast<sps::TilePlan*>(ws + l.k_plan);
  }
  a.seeds = backward ? reinterpret_cast<float*>(ws + l.seeds) : nullptr;
  a.B = B;
  a.H = H;
  a.div_bh = sps::make_fast_div((uint32_t)(B * H));
  a.div_b = sps::make_fast_div((uint32_t)B);
  a.div_h = sps::make_fast_div((uint32_t)H);
  a.m.family = family;
  a.m.P = family == SPS_FAMILY_REVERSE_SPS ? 1 : 0;
  a.m.N = N;
  // Distances never exceed N, so windows are clamped to [-1, N] (any negative window admits nothing
  // but the persistent diagonal); this keeps the interval arithmetic inside int range.
  a.m.window = window < -1 ? -1 : (window > N ? N : window);
  a.m.has_pkw = has_pkw ? 1 : 0;
  a.m.pkw = pkw < -1 ? -1 : (pkw > N ? N : pkw);
  a.m.has_docs = docs != nullptr;
  return SPS_OK;
}

}  // namespace

// Error reporting for the entry points defined in other translation units (hidden: not part of the
// library's exported interface).
extern "C" __attribute__((visibility("hidden"))) int sps_capi_fail(int code, const char* msg) {
  return fail(code, "%s", msg);
}

extern "C" __attribute__((visibility("hidden"))) void sps_capi_clear() { g_last_error.clear(); }

extern "C" {

const char* sps_version(void) { return "sps_attn 0.1.0 (gfx950)"; }

int sps_last_error(char* buf, size_t len) {
  if (buf && len > 0) {
    std::strncpy(buf, g_last_error.c_str(), len - 1);
    buf[len - 1] = '\0';
  }
  return (int)g_last_error.size();
}

size_t sps_attn_workspace_bytes(int family, int B, int H, int N, int has_docs, int backward) {
  if (B < 0 || H < 0 || N < 0) return 0;
  return attn_layout(family, B, H, N, has_docs, backward).total;
}

int sps_attn_fwd(int family, int B, int H, int N, int D, int dtype, const void* q, const int64_t* q_strides,
                 const void* k, const int64_t* k_strides, const void* v, const int64_t* v_strides, void* o,
                 const int64_t* o_strides, float* lse, const void* docs, int docs_dtype,
                 int64_t docs_stride_b, float sm_scale, int window, int has_pkw, int pkw, void* workspace,
                 size_t workspace_bytes, void* stream) {
  g_last_error.clear();
  sps::AttnArgs a;
  int rc = setup_common(a, family, B, H, N, docs, docs_dtype, docs_stride_b, window, has_pkw, pkw,
                        workspace, workspace_bytes, 0);
  if (rc) return rc;
  if (!supported_head_dim(D)) return fail(SPS_E_UNSUPPORTED, "head_dim %d not supported", D);
  if (dtype != SPS_DTYPE_BF16 && dtype != SPS_DTYPE_F16)
    return fail(SPS_E_UNSUPPORTED, "attention dtype code %d not supported (bf16, f16)", dtype);
  // Any finite scale is taken (zero and negative ones too); a NaN or infinite one would leave the
  // softmax undefined.
  if (!std::isfinite(sm_scale)) return fail(SPS_E_INVALID, "sm_scale must be finite");
  const int need = (int64_t)B * H * N > 0;
  if ((rc = check_tensor("q", q, q_strides, need, N, D)) || (rc = check_tensor("k", k, k_strides, need, N, D)) ||
      (rc = check_tensor("v", v, v_strides, need, N, D)) || (rc = check_tensor("o", o, o_strides, need, N, D)))
    return rc;
  if (need && !lse) return fail(SPS_E_INVALID, "lse: null pointer");
  if (!need) return SPS_OK;
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.out = static_cast<uint16_t*>(o);
  a.sq = strides(q_strides);
  a.sk = strides(k_strides);
  a.sv = strides(v_strides);
  a.sout = strides(o_strides);
  a.lse = lse;
  a.sm_scale = sm_scale;
  a.scale2 = sm_scale * 1.4426950408889634f;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (docs && (rc = hip_status(sps::launch_row_layout(a, s), "document prepass"))) return rc;
  return hip_status(sps::launch_attn_fwd(a, D, dtype == SPS_DTYPE_F16, s), "attention forward");
}

static int attn_bwd_impl(int passes, int family, int B, int H, int N, int D, int dtype, const void* q,
                         const int64_t* q_strides, const void* k, const int64_t* k_strides, const void* v,
                         const int64_t* v_strides, const void* o, const int64_t* o_strides, const void* dout,
                         const int64_t* dout_strides, const float* lse, void* dq, const int64_t* dq_strides,
                         void* dk, const int64_t* dk_strides, void* dv, const int64_t* dv_strides, const void* docs,
                         int docs_dtype, int64_t docs_stride_b, float sm_scale, int window, int has_pkw, int pkw,
                         void* workspace, size_t workspace_bytes, void* stream) {
  g_last_error.clear();
  if ((passes & (SPS_BWD_DQ | SPS_BWD_DKDV)) == 0 ||
      (passes & ~(SPS_BWD_DQ | SPS_BWD_DKDV | SPS_BWD_REUSE_LAYOUT)) != 0)
    return fail(SPS_E_INVALID, "backward pass selector %d is not SPS_BWD_DQ, SPS_BWD_DKDV or both (optionally "
                "with SPS_BWD_REUSE_LAYOUT)", passes);
  sps::AttnArgs a;
  int rc = setup_common(a, family, B, H, N, docs, docs_dtype, docs_stride_b, window, has_pkw, pkw,
                        workspace, workspace_bytes, 1);
  if (rc) return rc;
  if (!supported_head_dim(D)) return fail(SPS_E_UNSUPPORTED, "head_dim %d not supported", D);
  if (dtype != SPS_DTYPE_BF16 && dtype != SPS_DTYPE_F16)
    return fail(SPS_E_UNSUPPORTED, "attention dtype code %d not supported (bf16, f16)", dtype);
  // Any finite scale is taken (zero and negative ones too); a NaN or infinite one would leave the
  // softmax undefined.
  if (!std::isfinite(sm_scale)) return fail(SPS_E_INVALID, "sm_scale must be finite");
  const int need = (int64_t)B * H * N > 0;
  if ((rc = check_tensor("q", q, q_strides, need, N, D)) || (rc = check_tensor("k", k, k_strides, need, N, D)) ||
      (rc = check_tensor("v", v, v_strides, need, N, D)) || (rc = check_tensor("o", o, o_strides, need, N, D)) ||
      (rc = check_tensor("dout", dout, dout_strides, need, N, D)) || (rc = check_tensor("dq", dq, dq_strides, need, N, D)) ||
      (rc = check_tensor("dk", dk, dk_strides, need, N, D)) || (rc = check_tensor("dv", dv, dv_strides, need, N, D)))
    return rc;
  if (need && !lse) return fail(SPS_E_INVALID, "lse: null pointer");
  if (!need) return SPS_OK;
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.o = static_cast<const uint16_t*>(o);
  a.dO = static_cast<const uint16_t*>(dout);
  a.dq = static_cast<uint16_t*>(dq);
  a.dk = static_cast<uint16_t*>(dk);
  a.dv = static_cast<uint16_t*>(dv);
  a.sq = strides(q_strides);
  a.sk = strides(k_strides);
  a.sv = strides(v_strides);
  a.so = strides(o_strides);
  a.sdo = strides(dout_strides);
  a.sdq = strides(dq_strides);
  a.sdk = strides(dk_strides);
  a.sdv = strides(dv_strides);
  a.lse = const_cast<float*>(lse);
  a.sm_scale = sm_scale;
  a.scale2 = sm_scale * 1.4426950408889634f;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // The row layout is computed by the dQ pass and left in the workspace for the dK/dV pass.
  if (docs && (passes & SPS_BWD_DQ) && !(passes & SPS_BWD_REUSE_LAYOUT) &&
      (rc = hip_status(sps::launch_row_layout(a, s), "document prepass")))
    return rc;
  return hip_status(sps::launch_attn_bwd(a, D, dtype == SPS_DTYPE_F16, passes & (SPS_BWD_DQ | SPS_BWD_DKDV), s),
                    "attention backward");
}

}  // extern "C"

extern "C" {

int sps_attn_bwd(int family, int B, int H, int N, int D, int dtype, const void* q, const int64_t* q_strides,
                 const void* k, const int64_t* k_strides, const void* v, const int64_t* v_strides,
                 const void* o, const int64_t* o_strides, const void* dout, const int64_t* dout_strides,
                 const float* lse, void* dq, const int64_t* dq_strides, void* dk, const int64_t* dk_strides,
                 void* dv, const int64_t* dv_strides, const void* docs, int docs_dtype, int64_t docs_stride_b,
                 float sm_scale, int window, int has_pkw, int pkw, void* workspace, size_t workspace_bytes,
                 void* stream) {
  return attn_bwd_impl(SPS_BWD_DQ | SPS_BWD_DKDV, family, B, H, N, D, dtype, q, q_strides, k, k_strides, v,
                       v_strides, o, o_strides, dout, dout_strides, lse, dq, dq_strides, dk, dk_strides, dv,
                       dv_strides, docs, docs_dtype, docs_stride_b, sm_scale, window, has_pkw, pkw, workspace,
                       workspace_bytes, stream);
}

int sps_attn_bwd_pass(int pass, int family, int B, int H, int N, int D, int dtype, const void* q,
                      const int64_t* q_strides, const void* k, const int64_t* k_strides, const void* v,
                      const int64_t* v_strides, const void* o, const int64_t* o_strides, const void* dout,
                      const int64_t* dout_strides, const float* lse, void* dq, const int64_t* dq_strides, void* dk,
                      const int64_t* dk_strides, void* dv, const int64_t* dv_strides, const void* docs,
                      int docs_dtype, int64_t docs_stride_b, float sm_scale, int window, int has_pkw, int pkw,
                      void* workspace, size_t workspace_bytes, void* stream) {
  return attn_bwd_impl(pass, family, B, H, N, D, dtype, q, q_strides, k, k_strides, v, v_strides, o, o_strides,
                       dout, dout_strides, lse, dq, dq_strides, dk, dk_strides, dv, dv_strides, docs, docs_dtype,
                       docs_stride_b, sm_scale, window, has_pkw, pkw, workspace, workspace_bytes, stream);
}

int sps_attn_mask(int family, int B, int N, const void* docs, int docs_dtype, int64_t docs_stride_b, int window,
                  int has_pkw, int pkw, int schedule, uint8_t* mask, void* workspace, size_t workspace_bytes,
                  void* stream) {
  g_last_error.clear();
  sps::AttnArgs a;
  int rc = setup_common(a, family, B, 1, N, docs, docs_dtype, docs_stride_b, window, has_pkw, pkw, workspace,
                        workspace_bytes, 0);
  if (rc) return rc;
  if (schedule != 0 && schedule != 1) return fail(SPS_E_INVALID, "schedule must be 0 or 1");
  if ((int64_t)B * N == 0) return SPS_OK;
  if (!mask) return fail(SPS_E_INVALID, "mask: null pointer");
  a.mask_out = mask;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (docs && (rc = hip_status(sps::launch_row_layout(a, s), "document prepass"))) return rc;
  return hip_status(sps::launch_mask_dump(a, schedule, s), "mask dump");
}

static int kv_bytes(int kv_dtype) { return kv_dtype == SPS_DTYPE_F32 ? 4 : 2; }

static bool decode_head_dim(int D) { return D == 16 || D == 32 || D == 64 || D == 128 || D == 256; }

size_t sps_decode_workspace_bytes(int B, int H, int D, int nq, int kv_dtype, int n_seg, const int64_t* seg_scan) {
  if (!decode_head_dim(D) || B < 0 || H < 0 || n_seg < 0 || n_seg > sps::kMaxDecodeSegs) return 0;
  const int ck = sps::decode_chunk_keys(D, kv_bytes(kv_dtype));
  int64_t chunks = 0;
  for (int s = 0; s < n_seg; ++s) chunks += (seg_scan[s] + ck - 1) / ck;
  const size_t bytes = (size_t)B * H * chunks * nq * sps::decode_record_floats(D) * sizeof(float);
  return align_up(bytes);
}

}  // extern "C"

// Bytes of the length snapshot of sps_decode_kv_update (after the partial records, 256-byte aligned).
static size_t decode_snapshot_bytes(int B, int H) {
  return align_up((size_t)B * H * sps::kSnapWords * sizeof(int64_t));
}

// Validation and launch shared by sps_decode (caller's workspace) and sps_decode_static (the
// library's scratch array). `workspace` is only read after `workspace_bytes` has been checked.
static int decode_impl(int B, int H, int D, int nq, const void* q, int q_dtype, const int64_t* q_strides,
                       int kv_dtype, int n_seg, const void* const* seg_k, const int64_t* seg_k_strides,
                       const void* const* seg_v, const int64_t* seg_v_strides, const void* const* seg_len,
                       const int* seg_len_dtype, const int* seg_len_per_head, const int64_t* seg_scan, int n_extra,
                       const void* const* extra_k, const void* const* extra_v, int extra_dtype,
                       const int64_t* extra_strides, const int* extra_query_mask, float sm_scale, float* out,
                       const int64_t* out_strides, void* workspace, size_t workspace_bytes, void* stream,
                       const sps::KvUpdateArgs* upd = nullptr) {
  if (B < 0 || H < 0) return fail(SPS_E_INVALID, "negative size B=%d H=%d", B, H);
  if (nq != 1 && nq != 2) return fail(SPS_E_INVALID, "nq must be 1 or 2 (got %d)", nq);
  if (!decode_head_dim(D)) return fail(SPS_E_UNSUPPORTED, "decode head_dim %d not supported", D);
  if (kv_dtype != SPS_DTYPE_BF16 && kv_dtype != SPS_DTYPE_F16 && kv_dtype != SPS_DTYPE_F32)
    return fail(SPS_E_UNSUPPORTED, "K/V dtype code %d not supported", kv_dtype);
  if (q_dtype != SPS_DTYPE_BF16 && q_dtype != SPS_DTYPE_F16 && q_dtype != SPS_DTYPE_F32)
    return fail(SPS_E_UNSUPPORTED, "query dtype code %d not supported", q_dtype);
  if (n_extra > 0 && extra_dtype != SPS_DTYPE_BF16 && extra_dtype != SPS_DTYPE_F16 && extra_dtype != SPS_DTYPE_F32)
    return fail(SPS_E_UNSUPPORTED, "extra K/V dtype code %d not supported", extra_dtype);
  if (n_seg < 0 || n_seg > sps::kMaxDecodeSegs)
    return fail(SPS_E_INVALID, "at most %d segments (got %d)", sps::kMaxDecodeSegs, n_seg);
  if (n_extra < 0 || n_extra > sps::kMaxDecodeExtras)
    return fail(SPS_E_INVALID, "at most %d extra keys (got %d)", sps::kMaxDecodeExtras, n_extra);
  if ((int64_t)B * H == 0) return SPS_OK;
  if (!q || !q_strides || !out || !out_strides) return fail(SPS_E_INVALID, "q/out: null pointer");
  if (!(std::isfinite(sm_scale))) return fail(SPS_E_INVALID, "sm_scale must be finite");
  const size_t part_bytes = sps_decode_workspace_bytes(B, H, D, nq, kv_dtype, n_seg, seg_scan);
  const size_t need = part_bytes + (upd ? decode_snapshot_bytes(B, H) : 0);
  if (workspace_bytes < need) return fail(SPS_E_WORKSPACE, "workspace too small: %zu < %zu", workspace_bytes, need);
  sps::DecodeArgs a;
  std::memset(&a, 0, sizeof(a));
  a.B = B;
  a.H = H;
  a.NQ = nq;
  a.n_seg = n_seg;
  a.n_extra = n_extra;
  const int kb = kv_bytes(kv_dtype);
  const int epl = 16 / kb;
  const int ck = sps::decode_chunk_keys(D, kb);
  int chunk = 0;
  for (int s = 0; s < n_seg; ++s) {
    sps::DecodeSeg& sg = a.seg[s];
    if (seg_scan[s] < 0 || seg_scan[s] > INT32_MAX)
      return fail(SPS_E_INVALID, "segment %d: scan length %lld out of range", s, (long long)seg_scan[s]);
    sg.scan = (int)seg_scan[s];
    sg.chunk_base = chunk;
    chunk += (sg.scan + ck - 1) / ck;
    if (sg.scan == 0) continue;
    if (!seg_k[s] || !seg_v[s] || !seg_len[s]) return fail(SPS_E_INVALID, "segment %d: null pointer", s);
    if (!aligned16(seg_k[s]) || !aligned16(seg_v[s]))
      return fail(SPS_E_INVALID, "segment %d: K/V base must be 16-byte aligned", s);
    const int64_t* ks = seg_k_strides + 3 * s;
    const int64_t* vs = seg_v_strides + 3 * s;
    for (int i = 0; i < 3; ++i)
      if (ks[i] % epl != 0 || vs[i] % epl != 0)
        return fail(SPS_E_INVALID, "segment %d: strides must be multiples of 16 bytes", s);
    if (seg_len_dtype[s] != SPS_DTYPE_I32 && seg_len_dtype[s] != SPS_DTYPE_I64)
      return fail(SPS_E_INVALID, "segment %d: lengths must be int32 or int64", s);
    sg.k = seg_k[s];
    sg.v = seg_v[s];
    sg.ksb = ks[0];
    sg.ksh = ks[1];
    sg.kst = ks[2];
    sg.vsb = vs[0];
    sg.vsh = vs[1];
    sg.vst = vs[2];
    sg.len = seg_len[s];
    sg.len_i64 = seg_len_dtype[s] == SPS_DTYPE_I64;
    sg.len_per_head = seg_len_per_head[s] != 0;
  }
  // Segments with scan 0 own no chunk; give them a valid (never read) length pointer source.
  for (int s = 0; s < n_seg; ++s) {
    if (a.seg[s].scan == 0) {
      a.seg[s].len = nullptr;
    }
  }
  a.n_chunks = chunk;
  a.chunk_keys = ck;
  for (int e = 0; e < n_extra; ++e) {
    if (!extra_k[e] || !extra_v[e]) return fail(SPS_E_INVALID, "extra %d: null pointer", e);
    a.ek[e] = extra_k[e];
    a.ev[e] = extra_v[e];
    a.emask[e] = extra_query_mask[e];
  }
  if (n_extra > 0) {
    a.e_sb = extra_strides[0];
    a.e_sh = extra_strides[1];
  }
  a.e_dtype = extra_dtype;
  a.q_dtype = q_dtype;
  a.q = q;
  a.q_sb = q_strides[0];
  a.q_ss = q_strides[1];
  a.q_sh = q_strides[2];
  a.q_packed = q_dtype == kv_dtype && kv_dtype != SPS_DTYPE_F32 && aligned16(q) && D % 8 == 0 &&
               q_strides[0] % 8 == 0 && q_strides[1] % 8 == 0 && q_strides[2] % 8 == 0;
  a.out = out;
  a.o_sb = out_strides[0];
  a.o_ss = out_strides[1];
  a.o_sh = out_strides[2];
  a.scale2 = sm_scale * 1.4426950408889634f;
  a.part = static_cast<float*>(workspace);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (!upd) return hip_status(sps::launch_decode(a, D, kv_dtype, st), "decode");
  // The update folds into the launch when it copies 16-byte pieces (no dtype conversion, aligned rows)
  // and the grid has a first chunk for every (sequence, head) to take the length snapshot; otherwise
  // it runs as its own launch after the attention (same results).
  if (upd->vec16 && a.n_chunks > 0) {
    a.snap = reinterpret_cast<int64_t*>(static_cast<char*>(workspace) + part_bytes);
    a.upd = *upd;
    return hip_status(sps::launch_decode(a, D, kv_dtype, st), "decode with kv update");
  }
  const int rc = hip_status(sps::launch_decode(a, D, kv_dtype, st), "decode");
  if (rc) return rc;
  return hip_status(sps::launch_kv_update(*upd, st), "kv update");
}

// Scratch of sps_decode_static: the per-chunk partial records live in this array instead of a
// caller-provided workspace. Each GPU holds its own copy, at its own address, for the life of the
// process. In host code `decode_scratch` names a host-side stand-in, not device memory: its device
// address comes from hipGetSymbolAddress, once per device, on that device's first call.
constexpr size_t kDecodeScratchBytes = size_t(16) << 20;
static __device__ __align__(256) unsigned char decode_scratch[kDecodeScratchBytes];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of the current device's copy of decode_scratch.
int decode_scratch_ptr(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(SPS_E_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(SPS_E_UNSUPPORTED, "device %d: the scratch table covers devices 0..%d", dev, kMaxScratchDevices - 1);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(decode_scratch));
    if (e != hipSuccess || !p)
      return fail(SPS_E_HIP, "hipGetSymbolAddress(decode_scratch): %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SPS_OK;
}
}  // namespace

extern "C" {

int sps_decode(int B, int H, int D, int nq, const void* q, int q_dtype, const int64_t* q_strides, int kv_dtype,
               int n_seg, const void* const* seg_k, const int64_t* seg_k_strides, const void* const* seg_v,
               const int64_t* seg_v_strides, const void* const* seg_len, const int* seg_len_dtype,
               const int* seg_len_per_head, const int64_t* seg_scan, int n_extra, const void* const* extra_k,
               const void* const* extra_v, int extra_dtype, const int64_t* extra_strides,
               const int* extra_query_mask, float sm_scale, float* out, const int64_t* out_strides,
               void* workspace, size_t workspace_bytes, void* stream) {
  g_last_error.clear();
  return decode_impl(B, H, D, nq, q, q_dtype, q_strides, kv_dtype, n_seg, seg_k, seg_k_strides, seg_v,
                     seg_v_strides, seg_len, seg_len_dtype, seg_len_per_head, seg_scan, n_extra, extra_k, extra_v,
                     extra_dtype, extra_strides, extra_query_mask, sm_scale, out, out_strides, workspace,
                     workspace_bytes, stream);
}

int sps_decode_static(int B, int H, int D, int nq, const void* q, int q_dtype, const int64_t* q_strides,
                      int kv_dtype, int n_seg, const void* const* seg_k, const int64_t* seg_k_strides,
                      const void* const* seg_v, const int64_t* seg_v_strides, const void* const* seg_len,
                      const int* seg_len_dtype, const int* seg_len_per_head, const int64_t* seg_scan, int n_extra,
                      const void* const* extra_k, const void* const* extra_v, int extra_dtype,
                      const int64_t* extra_strides, const int* extra_query_mask, float sm_scale, float* out,
                      const int64_t* out_strides, void* stream) {
  g_last_error.clear();
  if (n_seg < 0 || n_seg > sps::kMaxDecodeSegs)
    return fail(SPS_E_INVALID, "at most %d segments (got %d)", sps::kMaxDecodeSegs, n_seg);
  if (n_seg > 0 && !seg_scan) return fail(SPS_E_INVALID, "seg_scan: null pointer");
  const size_t need = sps_decode_workspace_bytes(B, H, D, nq, kv_dtype, n_seg, seg_scan);
  if (need > kDecodeScratchBytes)
    return fail(SPS_E_UNSUPPORTED,
                "sps_decode_static: the partial records need %zu bytes, more than the %zu-byte scratch "
                "array (use sps_decode with a workspace)", need, kDecodeScratchBytes);
  void* ptr = nullptr;
  if ((int64_t)B * H > 0) {
    const int rc = decode_scratch_ptr(&ptr);
    if (rc) return rc;
  }
  return decode_impl(B, H, D, nq, q, q_dtype, q_strides, kv_dtype, n_seg, seg_k, seg_k_strides, seg_v,
                     seg_v_strides, seg_len, seg_len_dtype, seg_len_per_head, seg_scan, n_extra, extra_k, extra_v,
                     extra_dtype, extra_strides, extra_query_mask, sm_scale, out, out_strides, ptr,
                     kDecodeScratchBytes, stream);
}

}  // extern "C"

// Validates the arguments of a KV-cache update and fills its argument block (shared by
// sps_kv_update and sps_decode_kv_update). Returns SPS_OK, or an error with nothing launched; *empty
// is set when there is nothing to do (B * H * D == 0).
static int kv_update_setup(sps::KvUpdateArgs& a, bool* empty, int B, int H, int D, int kv_dtype, void* ring_k,
                           void* ring_v, const int64_t* ring_strides, int ring_storage, int window_tokens,
                           void* ring_len, void* ring_pos, const int64_t* ring_len_strides, void* ret_k, void* ret_v,
                           const int64_t* ret_strides, int ret_storage, void* ret_len,
                           const int64_t* ret_len_strides, int len_dtype, int new_dtype, const void* k_window,
                           const void* v_window, const void* k_retained, const void* v_retained,
                           const int64_t* new_strides, const void* active, int active_dtype, int64_t active_stride) {
  *empty = false;
  if (B < 0 || H < 0 || D < 0) return fail(SPS_E_INVALID, "negative size B=%d H=%d D=%d", B, H, D);
  auto float_type = [](int t) { return t == SPS_DTYPE_BF16 || t == SPS_DTYPE_F16 || t == SPS_DTYPE_F32; };
  if (!float_type(kv_dtype)) return fail(SPS_E_UNSUPPORTED, "cache dtype code %d not supported", kv_dtype);
  if (!float_type(new_dtype)) return fail(SPS_E_UNSUPPORTED, "new K/V dtype code %d not supported", new_dtype);
  if (len_dtype != SPS_DTYPE_I32 && len_dtype != SPS_DTYPE_I64)
    return fail(SPS_E_INVALID, "lengths must be int32 or int64 (dtype code %d)", len_dtype);
  int active_bytes = 0;
  if (active_dtype == SPS_DTYPE_U8) active_bytes = 1;
  else if (active_dtype == SPS_DTYPE_I32) active_bytes = 4;
  else if (active_dtype == SPS_DTYPE_I64) active_bytes = 8;
  else return fail(SPS_E_INVALID, "active mask must be bool/uint8, int32 or int64 (dtype code %d)", active_dtype);
  if (ret_storage < 0 || ring_storage < 0) return fail(SPS_E_INVALID, "negative cache storage");
  if ((int64_t)B * H * D == 0) {
    *empty = true;
    return SPS_OK;
  }
  if (!active || !ret_k || !ret_v || !ret_len || !k_retained || !v_retained || !ret_strides || !ret_len_strides ||
      !new_strides)
    return fail(SPS_E_INVALID, "retained cache / new K/V / active mask: null pointer");
  if (window_tokens > 0) {
    if (!ring_k || !ring_v || !ring_len || !ring_pos || !k_window || !v_window || !ring_strides || !ring_len_strides)
      return fail(SPS_E_INVALID, "ring cache: null pointer");
    if (window_tokens > ring_storage)
      return fail(SPS_E_INVALID, "window_tokens %d exceeds the ring storage %d", window_tokens, ring_storage);
  }
  std::memset(&a, 0, sizeof(a));
  a.B = B;
  a.H = H;
  a.D = D;
  a.kv_dtype = kv_dtype;
  a.new_dtype = new_dtype;
  a.window = window_tokens > 0 ? window_tokens : 0;
  if (a.window > 0) {
    a.ring_k = ring_k;
    a.ring_v = ring_v;
    a.rk_sb = ring_strides[0];
    a.rk_sh = ring_strides[1];
    a.rk_st = ring_strides[2];
    a.rv_sb = ring_strides[3];
    a.rv_sh = ring_strides[4];
    a.rv_st = ring_strides[5];
    a.ring_storage = ring_storage;
    a.ring_len = ring_len;
    a.ring_pos = ring_pos;
    a.ring_len_sb = ring_len_strides[0];
    a.ring_pos_sb = ring_len_strides[1];
    a.kw = k_window;
    a.vw = v_window;
    a.kw_sb = new_strides[0];
    a.kw_sh = new_strides[1];
    a.vw_sb = new_strides[2];
    a.vw_sh = new_strides[3];
  }
  a.ret_k = ret_k;
  a.ret_v = ret_v;
  a.tk_sb = ret_strides[0];
  a.tk_sh = ret_strides[1];
  a.tk_st = ret_strides[2];
  a.tv_sb = ret_strides[3];
  a.tv_sh = ret_strides[4];
  a.tv_st = ret_strides[5];
  a.ret_storage = ret_storage;
  a.ret_len = ret_len;
  a.ret_len_sb = ret_len_strides[0];
  a.ret_len_sh = ret_len_strides[1];
  a.len_i64 = len_dtype == SPS_DTYPE_I64;
  a.kr = k_retained;
  a.vr = v_retained;
  a.kr_sb = new_strides[4];
  a.kr_sh = new_strides[5];
  a.vr_sb = new_strides[6];
  a.vr_sh = new_strides[7];
  a.active = active;
  a.active_bytes = active_bytes;
  a.active_sb = active_stride;
  // 16-byte pieces when no conversion is needed and every row start is 16-byte aligned.
  const int64_t esz = kv_dtype == SPS_DTYPE_F32 ? 4 : 2;
  bool vec = new_dtype == kv_dtype && (D * esz) % 16 == 0 && H <= sps::kMaxVecHeads;
  const void* bases[] = {a.ret_k, a.ret_v, a.kr, a.vr, a.window > 0 ? a.ring_k : nullptr,
                         a.window > 0 ? a.ring_v : nullptr, a.window > 0 ? a.kw : nullptr,
                         a.window > 0 ? a.vw : nullptr};
  for (const void* p : bases) vec = vec && aligned16(p);
  const int64_t strides[] = {a.tk_sb, a.tk_sh, a.tk_st, a.tv_sb, a.tv_sh, a.tv_st, a.kr_sb, a.kr_sh, a.vr_sb,
                             a.vr_sh, a.rk_sb, a.rk_sh, a.rk_st, a.rv_sb, a.rv_sh, a.rv_st, a.kw_sb, a.kw_sh,
                             a.vw_sb, a.vw_sh};
  for (int64_t st : strides) vec = vec && (st * esz) % 16 == 0;
  a.vec16 = vec ? 1 : 0;
  return SPS_OK;
}


extern "C" {

int sps_kv_update(int B, int H, int D, int kv_dtype, void* ring_k, void* ring_v, const int64_t* ring_strides,
                  int ring_storage, int window_tokens, void* ring_len, void* ring_pos,
                  const int64_t* ring_len_strides, void* ret_k, void* ret_v, const int64_t* ret_strides,
                  int ret_storage, void* ret_len, const int64_t* ret_len_strides, int len_dtype, int new_dtype,
                  const void* k_window, const void* v_window, const void* k_retained, const void* v_retained,
                  const int64_t* new_strides, const void* active, int active_dtype, int64_t active_stride,
                  void* stream) {
  g_last_error.clear();
  sps::KvUpdateArgs a;
  bool empty = false;
  const int rc = kv_update_setup(a, &empty, B, H, D, kv_dtype, ring_k, ring_v, ring_strides, ring_storage,
                                 window_tokens, ring_len, ring_pos, ring_len_strides, ret_k, ret_v, ret_strides,
                                 ret_storage, ret_len, ret_len_strides, len_dtype, new_dtype, k_window, v_window,
                                 k_retained, v_retained, new_strides, active, active_dtype, active_stride);
  if (rc || empty) return rc;
  return hip_status(sps::launch_kv_update(a, static_cast<hipStream_t>(stream)), "kv update");
}

size_t sps_decode_kv_update_workspace_bytes(int B, int H, int D, int nq, int kv_dtype, int n_seg,
                                            const int64_t* seg_scan) {
  if (!decode_head_dim(D) || B < 0 || H < 0 || n_seg < 0 || n_seg > sps::kMaxDecodeSegs) return 0;
  return sps_decode_workspace_bytes(B, H, D, nq, kv_dtype, n_seg, seg_scan) + decode_snapshot_bytes(B, H);
}

int sps_decode_kv_update(int B, int H, int D, int nq, const void* q, int q_dtype, const int64_t* q_strides,
                         int kv_dtype, int n_seg, const void* const* seg_k, const int64_t* seg_k_strides,
                         const void* const* seg_v, const int64_t* seg_v_strides, const void* const* seg_len,
                         const int* seg_len_dtype, const int* seg_len_per_head, const int64_t* seg_scan,
                         int n_extra, const void* const* extra_k, const void* const* extra_v, int extra_dtype,
                         const int64_t* extra_strides, const int* extra_query_mask, float sm_scale, float* out,
                         const int64_t* out_strides, void* ring_k, void* ring_v, const int64_t* ring_strides,
                         int ring_storage, int window_tokens, void* ring_len, void* ring_pos,
                         const int64_t* ring_len_strides, void* ret_k, void* ret_v, const int64_t* ret_strides,
                         int ret_storage, void* ret_len, const int64_t* ret_len_strides, int len_dtype,
                         int new_dtype, const void* k_window, const void* v_window, const void* k_retained,
                         const void* v_retained, const int64_t* new_strides, const void* active, int active_dtype,
                         int64_t active_stride, void* workspace, size_t workspace_bytes, void* stream) {
  g_last_error.clear();
  sps::KvUpdateArgs u;
  bool empty = false;
  int rc = kv_update_setup(u, &empty, B, H, D, kv_dtype, ring_k, ring_v, ring_strides, ring_storage, window_tokens,
                           ring_len, ring_pos, ring_len_strides, ret_k, ret_v, ret_strides, ret_storage, ret_len,
                           ret_len_strides, len_dtype, new_dtype, k_window, v_window, k_retained, v_retained,
                           new_strides, active, active_dtype, active_stride);
  if (rc) return rc;
  if (n_seg > 0 && !seg_scan) return fail(SPS_E_INVALID, "seg_scan: null pointer");
  return decode_impl(B, H, D, nq, q, q_dtype, q_strides, kv_dtype, n_seg, seg_k, seg_k_strides, seg_v,
                     seg_v_strides, seg_len, seg_len_dtype, seg_len_per_head, seg_scan, n_extra, extra_k, extra_v,
                     extra_dtype, extra_strides, extra_query_mask, sm_scale, out, out_strides, workspace,
                     workspace_bytes, stream, empty ? nullptr : &u);
}

int sps_rope_qkv(int B, int N, int H, int D, int in_dtype, const void* q, const int64_t* q_strides, const void* k,
                 const int64_t* k_strides, const void* v, const int64_t* v_strides, const float* freqs,
                 const int64_t* freqs_strides, int out_dtype, void* q_out, const int64_t* q_out_strides,
                 void* k_out, const int64_t* k_out_strides, void* v_out, const int64_t* v_out_strides,
                 void* stream) {
  g_last_error.clear();
  if (B < 0 || N < 0 || H < 0 || D < 0) return fail(SPS_E_INVALID, "negative size B=%d N=%d H=%d D=%d", B, N, H, D);
  auto float_type = [](int t) { return t == SPS_DTYPE_BF16 || t == SPS_DTYPE_F16 || t == SPS_DTYPE_F32; };
  if (!float_type(in_dtype)) return fail(SPS_E_UNSUPPORTED, "input dtype code %d not supported", in_dtype);
  if (!float_type(out_dtype)) return fail(SPS_E_UNSUPPORTED, "output dtype code %d not supported", out_dtype);
  if (D % 8 != 0) return fail(SPS_E_UNSUPPORTED, "head_dim %d must be a multiple of 8", D);
  if ((int64_t)B * N * H * D == 0) return SPS_OK;
  if (!q || !k || !freqs || !q_out || !k_out || !q_strides || !k_strides || !freqs_strides || !q_out_strides ||
      !k_out_strides)
    return fail(SPS_E_INVALID, "q/k/freqs/outputs: null pointer");
  if (v && (!v_out || !v_strides || !v_out_strides)) return fail(SPS_E_INVALID, "v output: null pointer");
  // 16-byte pieces: every row start must be 16-byte aligned in every tensor.
  const int64_t in_el = in_dtype == SPS_DTYPE_F32 ? 4 : 2, out_el = out_dtype == SPS_DTYPE_F32 ? 4 : 2;
  auto rows_aligned = [](const void* p, const int64_t* st, int64_t el) {
    if (!aligned16(p)) return false;
    for (int i = 0; i < 3; ++i)
      if ((st[i] * el) % 16 != 0) return false;
    return true;
  };
  if (!rows_aligned(q, q_strides, in_el) || !rows_aligned(k, k_strides, in_el) ||
      (v && !rows_aligned(v, v_strides, in_el)))
    return fail(SPS_E_INVALID, "q/k/v rows must start 16-byte aligned (base and strides)");
  if (!rows_aligned(q_out, q_out_strides, out_el) || !rows_aligned(k_out, k_out_strides, out_el) ||
      (v && !rows_aligned(v_out, v_out_strides, out_el)))
    return fail(SPS_E_INVALID, "output rows must start 16-byte aligned (base and strides)");
  if (!aligned16(freqs) || (freqs_strides[0] * 4) % 16 != 0 || (freqs_strides[1] * 4) % 16 != 0)
    return fail(SPS_E_INVALID, "freqs rows must start 16-byte aligned");
  sps::RopeArgs a;
  std::memset(&a, 0, sizeof(a));
  a.B = B;
  a.N = N;
  a.H = H;
  a.D = D;
  a.in_dtype = in_dtype;
  a.out_dtype = out_dtype;
  a.q = q;
  a.k = k;
  a.v = v;
  a.q_sb = q_strides[0], a.q_sn = q_strides[1], a.q_sh = q_strides[2];
  a.k_sb = k_strides[0], a.k_sn = k_strides[1], a.k_sh = k_strides[2];
  if (v) a.v_sb = v_strides[0], a.v_sn = v_strides[1], a.v_sh = v_strides[2];
  a.freqs = freqs;
  a.f_sb = freqs_strides[0];
  a.f_sn = freqs_strides[1];
  a.qo = q_out;
  a.ko = k_out;
  a.vo = v_out;
  a.qo_sb = q_out_strides[0], a.qo_sn = q_out_strides[1], a.qo_sh = q_out_strides[2];
  a.ko_sb = k_out_strides[0], a.ko_sn = k_out_strides[1], a.ko_sh = k_out_strides[2];
  if (v) a.vo_sb = v_out_strides[0], a.vo_sn = v_out_strides[1], a.vo_sh = v_out_strides[2];
  return hip_status(sps::launch_rope_qkv(a, static_cast<hipStream_t>(stream)), "rope");
}

int sps_prefill_to_decode(int B, int T, int H, int D, int in_dtype, const void* k, const int64_t* k_strides,
                          const void* v, const int64_t* v_strides, int window_slot, int retained_slot,
                          const uint8_t* doc_mask, int64_t doc_mask_stride, int kv_dtype, void* ring_k,
                          void* ring_v, const int64_t* ring_strides, int ring_storage, int window_tokens,
                          void* ring_len, void* ring_pos, const int64_t* ring_len_strides, void* ret_k,
                          void* ret_v, const int64_t* ret_strides, int ret_storage, void* ret_len,
                          const int64_t* ret_len_strides, int len_dtype, void* stream) {
  g_last_error.clear();
  if (B < 0 || T < 0 || H < 0 || D < 0) return fail(SPS_E_INVALID, "negative size B=%d T=%d H=%d D=%d", B, T, H, D);
  auto float_type = [](int t) { return t == SPS_DTYPE_BF16 || t == SPS_DTYPE_F16 || t == SPS_DTYPE_F32; };
  if (!float_type(in_dtype)) return fail(SPS_E_UNSUPPORTED, "K/V dtype code %d not supported", in_dtype);
  if (!float_type(kv_dtype)) return fail(SPS_E_UNSUPPORTED, "cache dtype code %d not supported", kv_dtype);
  if (len_dtype != SPS_DTYPE_I32 && len_dtype != SPS_DTYPE_I64)
    return fail(SPS_E_INVALID, "lengths must be int32 or int64 (dtype code %d)", len_dtype);
  if (D % 8 != 0 || D > 8 * 256) return fail(SPS_E_UNSUPPORTED, "head_dim %d must be a multiple of 8", D);
  if ((window_slot != 0 && window_slot != 1) || (retained_slot != 0 && retained_slot != 1))
    return fail(SPS_E_INVALID, "slot indices must be 0 or 1");
  if (ret_storage < 0 || ring_storage < 0) return fail(SPS_E_INVALID, "negative cache storage");
  if ((int64_t)B * T * H * D == 0) return SPS_OK;
  if (!k || !v || !doc_mask || !ret_k || !ret_v || !ret_len || !k_strides || !v_strides || !ret_strides ||
      !ret_len_strides)
    return fail(SPS_E_INVALID, "K/V, mask or retained cache: null pointer");
  if (window_tokens > 0 && (!ring_k || !ring_v || !ring_len || !ring_pos || !ring_strides || !ring_len_strides))
    return fail(SPS_E_INVALID, "ring cache: null pointer");
  if (window_tokens > ring_storage && window_tokens > 0)
    return fail(SPS_E_INVALID, "window_tokens %d exceeds the ring storage %d", window_tokens, ring_storage);
  const int64_t in_el = in_dtype == SPS_DTYPE_F32 ? 4 : 2, kv_el = kv_dtype == SPS_DTYPE_F32 ? 4 : 2;
  auto aligned_rows = [](const void* p, const int64_t* st, int n, int64_t el) {
    if (!aligned16(p)) return false;
    for (int i = 0; i < n; ++i)
      if ((st[i] * el) % 16 != 0) return false;
    return true;
  };
  if (!aligned_rows(k, k_strides, 3, in_el) || !aligned_rows(v, v_strides, 3, in_el))
    return fail(SPS_E_INVALID, "K/V rows must start 16-byte aligned (base and strides)");
  if (!aligned_rows(ret_k, ret_strides, 3, kv_el) || !aligned_rows(ret_v, ret_strides + 3, 3, kv_el) ||
      (window_tokens > 0 &&
       (!aligned_rows(ring_k, ring_strides, 3, kv_el) || !aligned_rows(ring_v, ring_strides + 3, 3, kv_el))))
    return fail(SPS_E_INVALID, "cache rows must start 16-byte aligned (base and strides)");
  sps::PrefillStateArgs a;
  std::memset(&a, 0, sizeof(a));
  a.B = B;
  a.T = T;
  a.H = H;
  a.D = D;
  a.in_dtype = in_dtype;
  a.kv_dtype = kv_dtype;
  a.k = k;
  a.v = v;
  a.k_sb = k_strides[0], a.k_sn = k_strides[1], a.k_sh = k_strides[2];
  a.v_sb = v_strides[0], a.v_sn = v_strides[1], a.v_sh = v_strides[2];
  a.window_slot = window_slot;
  a.retained_slot = retained_slot;
  a.mask = doc_mask;
  a.mask_sb = doc_mask_stride;
  a.window = window_tokens > 0 ? window_tokens : 0;
  if (a.window > 0) {
    a.ring_k = ring_k;
    a.ring_v = ring_v;
    a.rk_sb = ring_strides[0], a.rk_sh = ring_strides[1], a.rk_st = ring_strides[2];
    a.rv_sb = ring_strides[3], a.rv_sh = ring_strides[4], a.rv_st = ring_strides[5];
    a.ring_storage = ring_storage;
    a.ring_len = ring_len;
    a.ring_pos = ring_pos;
    a.ring_len_sb = ring_len_strides[0];
    a.ring_pos_sb = ring_len_strides[1];
  }
  a.ret_k = ret_k;
  a.ret_v = ret_v;
  a.tk_sb = ret_strides[0], a.tk_sh = ret_strides[1], a.tk_st = ret_strides[2];
  a.tv_sb = ret_strides[3], a.tv_sh = ret_strides[4], a.tv_st = ret_strides[5];
  a.ret_storage = ret_storage;
  a.ret_len = ret_len;
  a.ret_len_sb = ret_len_strides[0];
  a.ret_len_sh = ret_len_strides[1];
  a.len_i64 = len_dtype == SPS_DTYPE_I64;
  return hip_status(sps::launch_prefill_state(a, static_cast<hipStream_t>(stream)), "prefill state");
}

}  // extern "C"
