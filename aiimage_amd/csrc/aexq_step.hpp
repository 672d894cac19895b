// The fused decode step's host/device definitions (aexq_step.hip, launched by
// aexq_decoder_run in aexq_api.hip); not part of the ABI.
#pragma once

#include "aexq_internal.hpp"

namespace aexq {

// The decoder layers of a decode step as one persistent launch (aexq_step.hip).
constexpr int kStepThreads = 768;       // threads per workgroup: 9 compute, 1 store, 2 poll waves
constexpr int kStepComputeWaves = 9;
constexpr int kStepOutWords = 1024;     // a workgroup's outputs of one phase, staged in LDS
constexpr int kStepHeadDim = 128;
constexpr int kStepMaxHidden = 1024;    // LDS rows sized for these maxima
constexpr int kStepMaxQ = 2048;
constexpr int kStepMaxInter = 4096;
constexpr int kStepMaxLayers = 64;      // the layer table is staged in LDS
constexpr int kStepMaxSplitPos = 64;    // cached positions per attention workgroup (8 waves x 8)
constexpr int kStepMaxSplits = 32;      // attention workgroups per kv head
constexpr int kStepMaxMerge = 32;       // output dims per merging workgroup
constexpr int kStepPartStride = 132;    // words per (q head, split) partial: m, l, 2 pad, acc[128]
// Copies of each vector exchange buffer: every producer writes all of them and
// workgroup b polls copy b % kStepReplicas, so the grid's polls of one vector
// spread over that many 4 KB pages (memory channels) instead of meeting on one.
constexpr int kStepReplicas = 8;
// The SwiGLU output (28 words per workgroup at the benchmark's shapes) in 4
// copies: its producers' stores of 8 copies take four store instructions, and
// 4 copies measured faster.
constexpr int kStepReplicasH = 4;
// Words between two copies of a vector of `words` words: whole 4 KB pages, an
// odd count of them (3 for 12 KB, 5 for 14 KB), so that the copies' first
// pages do not all fall on pages of one parity.
constexpr int step_replica_stride(int words) {
  return (((words + 1023) / 1024) | 1) * 1024;
}

// One decoder layer's device operands (Q4 codes and scales of q, k, v, o,
// gate, up, down; the two RMSNorm gammas; the layer's fp16 K/V caches
// [heads_kv][capacity][128]).
struct StepLayer {
  const uint32_t* w[7];
  const void* s[7];
  const float* g_attn;
  const float* g_mlp;
  uint16_t* kc;  // fp16 bits
  uint16_t* vc;
};

struct StepParams {
  const StepLayer* layers;  // device array [nlayers]
  int nlayers;
  int hidden, qw, kvw, inter, hq, hkv, cap;
  int fmt, gmode;           // layer weights: kQ4 with kG32 / kG16 scale groups, or kQ8 per row
  int sf16;                 // layer scales fp16 (else fp32)
  float eps, scale;
  const uint32_t* emb_codes;  // tied Q8 table [vocab][hidden] (device bytes q + 128)
  const void* emb_scales;
  int emb_sf16, vocab;
  const int32_t* token;     // device: this step's input token
  const int32_t* pos;       // device: this step's position (the new cache row)
  const float* cos_t;       // [cap][64]
  const float* sin_t;
  // exchange buffers of tagged words (see aexq_step.hip); the vectors every
  // workgroup polls are kStepReplicas copies (the SwiGLU output
  // kStepReplicasH) `*_rs` words apart
  uint32_t* xa_t;           // [kStepReplicas][xa_rs >= hidden]
  uint32_t* qkv_t;          // [kStepReplicas][qkv_rs >= qw + 2 kvw]
  uint32_t* part_t;         // [hq][splits][kStepPartStride] (one copy)
  uint32_t* attn_t;         // [kStepReplicas][attn_rs >= qw]
  uint32_t* xb_t;           // [kStepReplicas][xb_rs >= hidden]
  uint32_t* h_t;            // [kStepReplicasH][h_rs >= inter]
  int xa_rs, qkv_rs, attn_rs, xb_rs, h_rs;
  uint32_t* epoch;          // launch epoch counter
  int* err;                 // set when a wait exceeded its spin bound
  uint16_t* out;            // final hidden state, fp16 bits [hidden]
  // partition over the grid
  int rows_qkv, rows_hid, rows_inter;  // rows (pairs) per workgroup
  int splits, split_pos;               // attention workgroups per kv head, positions each
  int merge_dims;                      // output dims per merging workgroup
};
// Whether the fused step has a kernel for the layer format (fmt, gmode), q
// heads per kv head `gq` and the 16-byte code chunks (32 Q4 or 16 Q8 codes) per
// row of the hidden, q and intermediate widths.
bool decode_layers_supported(int fmt, int gmode, int gq, int ch_hidden, int ch_q, int ch_inter);
hipError_t decode_layers_launch(const StepParams& p, int grid, hipStream_t stream);
// Resident workgroups per CU of the fused step's kernel for a layer format.
hipError_t decode_layers_occupancy(int fmt, int gmode, int* per_cu);

}  // namespace aexq
