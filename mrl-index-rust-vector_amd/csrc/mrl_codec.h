// mrl_codec.h -- host-side ingest helpers shared by the C ABI and the synthetic generator.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <functional>

namespace mrl {

struct EdenFitView {
  uint32_t dim;
  uint32_t bits;
  uint64_t seed;
  const float* mean;
};

float f16_to_f32(uint16_t h);
uint16_t f32_to_f16(float f);
uint32_t crc32(const uint8_t* p, size_t n);
bool block_crc_ok(const uint8_t* block);
const float* lloyd_max(int bits, int* n);

// Cluster-grouped layout (no reference counterpart): a block whose rows all
// belong to one coarse cluster below 65536 records it in coarse_cluster_id
// (header bytes 12-13) and sets kBlockFlagOneCluster in block_flags (bytes
// 14-15); kNoCluster leaves both zero, as the reference's encoder does.
constexpr uint32_t kNoCluster = 0xffffffffu;
int encode_block(const float* vecs, uint32_t n, uint32_t dims, const uint32_t* ts, const uint32_t* src,
                 const EdenFitView* eden, const EdenFitView* eden_mid, uint8_t* block, uint32_t cluster = kNoCluster);
// The cluster of a block of n rows with per-row clusters c (kNoCluster unless
// they all agree on one below 65536).
uint32_t block_cluster(const uint32_t* c, uint64_t n);
int encode_corpus(const float* matrix, uint64_t n, uint32_t dims, uint32_t default_source,
                  const EdenFitView* eden, const EdenFitView* eden_mid, int n_threads, uint8_t* out,
                  const uint32_t* cluster = nullptr);
int eden_fit_band(const float* rows, uint64_t n_rows, uint32_t stride, uint32_t start, uint32_t dim, float* mean);
int parallel_for(uint64_t n, int n_threads, const std::function<void(uint64_t, uint64_t)>& fn);

// Synthetic corpus description (benchmark inputs).
struct SynthSpec {
  uint64_t n_docs;
  uint32_t dims;
  float mean_offset;       // added to every coordinate before normalising
  uint64_t seed;           // documents
  uint32_t n_centroids;    // 0: independent documents; else clustered
  uint64_t seed_centroids;
  uint64_t seed_assign;
  float noise_sigma;       // clustered: isotropic noise norm around the centroid
};

void gaussian_row(uint64_t seed, uint64_t stream, uint64_t row, uint32_t n, float* out);
void synth_doc(const SynthSpec& s, uint64_t row, float* out);
// The centroid of row `row` of a clustered corpus.
uint32_t synth_cluster(const SynthSpec& s, uint64_t row);
void synth_query(const SynthSpec& s, uint64_t seed_q, float noise_sigma, int fresh, uint64_t qi, float* out,
                 uint64_t* src_row);

}  // namespace mrl
