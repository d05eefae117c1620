/*
 * CPU oracle of the SPS attention visibility predicate. TEST INFRASTRUCTURE ONLY: used by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg as a checker; never by the product path.
 *
 * Restates the mask of the reference kernels (lil-lab/sps, src/modeling/models/attention/):
 *   document mask   docs[q] == docs[k]                     triton_sps_flash_attention.py:81-87
 *   temporary keys  q_tok - k_tok <= window (in tokens)    triton_sps_flash_attention.py:89-95
 *   persistent key  parity P (0: sps, 1: reverse_sps)      triton_sps_flash_attention.py:97,
 *                                                          triton_reverse_sps_flash_attention.py:123
 *   persistent-key window  q_tok - k_tok <= pkw            triton_sps_flash_attention.py:102-104
 *   self-persistent exemption (q == k)                     triton_sps_flash_attention.py:106-107
 *   causal          k <= q                                 triton_sps_flash_attention.py:109-111
 *   full family: causal and document mask only             triton_full_flash_attention.py:95-104
 * The reference applies these as finite additive biases (-1e6); a biased entry contributes
 * exp2(-1e6 * log2e) == 0 to any row that has an unbiased entry, and the diagonal is always
 * unbiased, so the boolean predicate below is the exact contract.
 *
 * Build: see oracle/Makefile (gcc, no dependencies).
 */
#include <stdint.h>
#include <string.h>

/* family: 0 full, 1 sps (persistent parity 0), 2 reverse_sps (persistent parity 1). */
int sps_oracle_visible(int family, int64_t q, int64_t k, int has_docs, int64_t doc_q, int64_t doc_k,
                       int64_t window, int has_pkw, int64_t pkw) {
  if (k > q) return 0;
  if (has_docs && doc_q != doc_k) return 0;
  if (family == 0) return 1;
  {
    const int persistent_parity = family == 2 ? 1 : 0;
    const int64_t q_tok = q / 2, k_tok = k / 2;
    if ((k % 2) == persistent_parity) {
      if (!has_pkw) return 1;
      if (q == k) return 1;
      return (q_tok - k_tok) <= pkw;
    }
    return (q_tok - k_tok) <= window;
  }
}

/* Full [n, n] mask (row = query) for one batch row; docs may be NULL. */
void sps_oracle_mask(int family, int64_t n, const int64_t* docs, int64_t window, int has_pkw, int64_t pkw,
                     uint8_t* out) {
  int64_t q, k;
  memset(out, 0, (size_t)(n * n));
  for (q = 0; q < n; ++q) {
    for (k = 0; k <= q; ++k) {
      const int hd = docs != 0;
      out[q * n + k] = (uint8_t)sps_oracle_visible(family, q, k, hd, hd ? docs[q] : 0, hd ? docs[k] : 0,
                                                   window, has_pkw, pkw);
    }
  }
}

/* Number of visible (query, key) pairs of one batch row (the useful-pair count). */
int64_t sps_oracle_count(int family, int64_t n, const int64_t* docs, int64_t window, int has_pkw, int64_t pkw) {
  int64_t q, k, total = 0;
  for (q = 0; q < n; ++q) {
    for (k = 0; k <= q; ++k) {
      const int hd = docs != 0;
      total += sps_oracle_visible(family, q, k, hd, hd ? docs[q] : 0, hd ? docs[k] : 0, window, has_pkw, pkw);
    }
  }
  return total;
}
