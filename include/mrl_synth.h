/*
 * mrl_synth.h -- seeded synthetic corpora for benchmarks and tests.
 *
 * No counterpart in the reference's scan API: it plays the role of the
 * reference's own synthetic bench setup (src/bin/mrl_index.rs:618-676 and
 * benches/scan_bench.rs:10-32: seeded Gaussian rows, L2-normalised, encoded
 * into PaxBlock64 blocks), with the generators the benchmark configurations
 * describe.  Row r depends only on (seed, r), so corpora can be generated in
 * parallel and in pieces.
 */
#ifndef MRL_SYNTH_H
#define MRL_SYNTH_H

#include <stdint.h>

#include "mrl_scan.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mrl_synth_spec {
  uint64_t n_docs;
  uint32_t dims;
  float mean_offset;       /* x_d = (1+d)^-1/2 z_d + mean_offset, then L2-normalised */
  uint64_t seed;
  uint32_t n_centroids;    /* 0: independent rows; else row = centroid + noise, renormalised */
  uint64_t seed_centroids;
  uint64_t seed_assign;
  float noise_sigma;       /* clustered rows: noise norm (per-dim sigma / sqrt(dims)) */
} mrl_synth_spec;

/* Rows [first_row, first_row + n_rows) into out (row-major). */
int mrl_synth_docs(const mrl_synth_spec *spec, uint64_t first_row, uint64_t n_rows, int n_threads, float *out);
/* fresh != 0: queries drawn like documents with seed_q.  Otherwise each query
 * is a document chosen uniformly (seeded) plus isotropic noise of norm
 * noise_sigma, renormalised; out_src_rows (may be NULL) gets that document. */
int mrl_synth_queries(const mrl_synth_spec *spec, uint64_t seed_q, float noise_sigma, int fresh, uint32_t n_q,
                      float *out, uint64_t *out_src_rows);
/* EdenFit::fit_prefix over the first n_rows documents (src/eden.rs:122-159). */
int mrl_synth_eden_fit(const mrl_synth_spec *spec, uint64_t n_rows, float *out_mean64);
/* Generate and encode all documents: ceil(n_docs/64) blocks, timestamp = row. */
int mrl_synth_encode(const mrl_synth_spec *spec, const mrl_eden_fit *eden, const mrl_eden_fit *eden_mid,
                     uint32_t default_source, int n_threads, void *out_blocks);
/* The same documents of a clustered corpus in the cluster-grouped layout
 * (mrl_encode_corpus_clustered): rows ordered by (centroid, row), timestamp
 * = position in that order; out_rows[p] (may be NULL) = the row at
 * position p. */
int mrl_synth_encode_clustered(const mrl_synth_spec *spec, const mrl_eden_fit *eden, const mrl_eden_fit *eden_mid,
                               uint32_t default_source, int n_threads, void *out_blocks, uint64_t *out_rows);

#ifdef __cplusplus
}
#endif
#endif
