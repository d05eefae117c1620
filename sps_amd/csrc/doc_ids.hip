// Document ids of token rows, one launch for the batch (one 1024-thread workgroup per row).
//
// Semantics (generate_left_padded_document_idx, model.py:70-99, and the interleaving of the SPS
// callers, reverse_sps/core.py:218-227): a token is real when it differs from the pad id. Rows must
// be left padded: a pad token after a real one marks the row invalid (the host raises). A real token's
// id is the row's pad count plus the number of real EOS tokens strictly before it (a document ends
// after its EOS); the i-th pad token gets id i, so left pads form one-token documents disjoint from
// the real suffix. With repeat = 2 every id is written twice (positions 2t and 2t + 1 of the
// interleaved input/<predict> sequence).
//
// The row is walked in tiles of 1024 tokens (one per thread, coalesced loads). Per tile, one block
// scan gives each token the number of pads and of real EOS tokens before it within the tile; running
// totals carry across tiles. A pad at position t is valid iff every token before it is a pad, i.e.
// iff the pads before it number exactly t, so validation needs no extra pass. The pad count of the
// whole row is needed by every real token's id, so the counts are taken in a first sweep and the ids
// written in a second one (both sweeps read the row; rows are short next to the attention they feed).
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sps {

constexpr int kIdThreads = 1024;
constexpr int kIdWaves = kIdThreads / 64;

struct DocIdArgs {
  const void* tokens;  // [B, T] int32 / int64
  int tok_i64;
  int64_t tok_sb;
  int64_t eos, pad;
  int B, T, repeat;
  void* out;  // [B, T * repeat] int32 / int64
  int out_i64;
  int64_t out_sb;
  int* bad;  // [B] 1 when the row has a pad after a real token (may be null)
};

__device__ __forceinline__ int64_t load_tok(const DocIdArgs& a, int b, int t) {
  if (a.tok_i64) return reinterpret_cast<const int64_t*>(a.tokens)[b * a.tok_sb + t];
  return reinterpret_cast<const int32_t*>(a.tokens)[b * a.tok_sb + t];
}

// Exclusive prefix sums over the workgroup of two counters packed in one 64-bit value (high word:
// real EOS, low word: pads; each below 2^31), and their workgroup total.
__device__ __forceinline__ uint64_t block_scan_pair(uint64_t x, uint64_t* s_tot, uint64_t& total) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint64_t inc = x;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint64_t y = __shfl_up(inc, o);
    if (lane >= o) inc += y;
  }
  if (lane == 63) s_tot[wave] = inc;
  __syncthreads();
  uint64_t before = 0;
  total = 0;
#pragma unroll
  for (int w = 0; w < kIdWaves; ++w) {
    const uint64_t v = s_tot[w];
    before += w < wave ? v : 0;
    total += v;
  }
  __syncthreads();  // s_tot is reused by the next tile
  return before + inc - x;
}

__global__ __launch_bounds__(kIdThreads) void doc_ids_kernel(const DocIdArgs a) {
  __shared__ uint64_t s_tot[kIdWaves];
  const int b = blockIdx.x, tid = threadIdx.x;
  // Sweep 1: pad count of the row and validity.
  uint64_t run = 0;  // (real EOS << 32) | pads, before the current tile
  bool bad = false;
  for (int t0 = 0; t0 < a.T; t0 += kIdThreads) {
    const int t = t0 + tid;
    const bool in = t < a.T;
    const int64_t tok = in ? load_tok(a, b, t) : a.pad;
    const bool is_pad = tok == a.pad;
    const uint64_t x = in ? (is_pad ? 1ull : 0ull) : 0ull;
    uint64_t total;
    const uint64_t ex = block_scan_pair(x, s_tot, total);
    const uint32_t pads_before = (uint32_t)(run + ex);
    bad |= in && is_pad && pads_before != (uint32_t)t;
    run += total;
  }
  const uint32_t row_pads = (uint32_t)run;
  const int any_bad = __syncthreads_or(bad);
  if (tid == 0 && a.bad) a.bad[b] = any_bad;
  // Sweep 2: ids.
  run = 0;
  for (int t0 = 0; t0 < a.T; t0 += kIdThreads) {
    const int t = t0 + tid;
    const bool in = t < a.T;
    const int64_t tok = in ? load_tok(a, b, t) : a.pad;
    const bool is_pad = tok == a.pad;
    const bool real_eos = !is_pad && tok == a.eos;
    const uint64_t x = in ? (is_pad ? 1ull : (real_eos ? (1ull << 32) : 0ull)) : 0ull;
    uint64_t total;
    const uint64_t ex = run + block_scan_pair(x, s_tot, total);
    run += total;
    if (!in) continue;
    const int64_t id = is_pad ? (int64_t)(uint32_t)ex : (int64_t)row_pads + (int64_t)(ex >> 32);
    for (int r = 0; r < a.repeat; ++r) {
      const int64_t at = b * a.out_sb + (int64_t)t * a.repeat + r;
      if (a.out_i64)
        reinterpret_cast<int64_t*>(a.out)[at] = id;
      else
        reinterpret_cast<int32_t*>(a.out)[at] = (int32_t)id;
    }
  }
}

hipError_t launch_doc_ids(const DocIdArgs& a, hipStream_t stream) {
  if (a.B == 0 || a.T == 0) return hipSuccess;
  hipLaunchKernelGGL(doc_ids_kernel, dim3(a.B), dim3(kIdThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace sps

// Declared in include/sps_attn.h; argument checks live here so the whole entry point is in one file.
#include "../../include/sps_attn.h"

extern "C" int sps_capi_fail(int code, const char* msg);
extern "C" void sps_capi_clear();

extern "C" int sps_document_ids(int B, int T, const void* tokens, int tokens_dtype, int64_t tokens_stride_b,
                                int64_t eos_token_id, int64_t pad_token_id, int repeat, void* out, int out_dtype,
                                int64_t out_stride_b, int* bad_rows, void* stream) {
  sps_capi_clear();
  if (B < 0 || T < 0) return sps_capi_fail(SPS_E_INVALID, "sps_document_ids: negative size");
  if (repeat != 1 && repeat != 2) return sps_capi_fail(SPS_E_INVALID, "sps_document_ids: repeat must be 1 or 2");
  if (tokens_dtype != SPS_DTYPE_I32 && tokens_dtype != SPS_DTYPE_I64)
    return sps_capi_fail(SPS_E_UNSUPPORTED, "sps_document_ids: token ids must be int32 or int64");
  if (out_dtype != SPS_DTYPE_I32 && out_dtype != SPS_DTYPE_I64)
    return sps_capi_fail(SPS_E_UNSUPPORTED, "sps_document_ids: document ids must be int32 or int64");
  if ((int64_t)T * repeat > INT32_MAX) return sps_capi_fail(SPS_E_UNSUPPORTED, "sps_document_ids: row too long");
  if ((int64_t)B * T == 0) return SPS_OK;
  if (!tokens || !out) return sps_capi_fail(SPS_E_INVALID, "sps_document_ids: null pointer");
  if (tokens_stride_b < T || out_stride_b < (int64_t)T * repeat)
    return sps_capi_fail(SPS_E_INVALID, "sps_document_ids: row stride shorter than the row");
  sps::DocIdArgs a;
  a.tokens = tokens;
  a.tok_i64 = tokens_dtype == SPS_DTYPE_I64;
  a.tok_sb = tokens_stride_b;
  a.eos = eos_token_id;
  a.pad = pad_token_id;
  a.B = B;
  a.T = T;
  a.repeat = repeat;
  a.out = out;
  a.out_i64 = out_dtype == SPS_DTYPE_I64;
  a.out_sb = out_stride_b;
  a.bad = bad_rows;
  const hipError_t e = sps::launch_doc_ids(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return sps_capi_fail(SPS_E_HIP, hipGetErrorString(e));
  return SPS_OK;
}
