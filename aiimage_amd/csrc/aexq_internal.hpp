// Shared host/device definitions of the aexq HIP library (not part of the ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace aexq {

constexpr int kMaxGroup = 8;  // matrices per grouped launch
constexpr int kWaves = 4;     // waves per workgroup of the matvec kernels
constexpr int kThreads = 64 * kWaves;
// logits (rows x M) one workgroup of the streaming LM head holds in LDS until
// its tile loop ends; the host sizes the grid so that no workgroup has more
constexpr int kArgLogitsMax = 2048;

enum Fmt : int { kQ8 = 0, kQ4 = 1 };

// Flags inside QmvParams::flags.
enum : int {
  kFlagRms = 1,        // RMSNorm-in prologue
  kFlagResidual = 2,   // y += residual
  kFlagYf32 = 4,       // output is fp32 (else fp16)
  kFlagAlphaIn = 8,    // alpha * (beta*C + sum) (Pack4 linear); else beta*C + alpha*sum (tiled)
  kFlagScaleF16 = 16,  // scales are fp16 (else fp32)
  kFlagXf32 = 32,      // activations fp32 (generic kernel only)
  kFlagXShared = 64,   // M = 1 streaming RMSNorm-in: every tile multiplies the same row
  kFlagArgF16 = 128,   // LM head: the argmax compares logits rounded to fp16 (ARGBHalf texture)
};

// Scale granularity of a streaming kernel: one per row (Q8), per 16 codes
// (the reference's shipping Q4), or per multiple of 32 codes (incl. per row).
enum GMode : int { kGRow = 0, kG16 = 1, kG32 = 2 };

// One matrix of a grouped launch; pointers are for batch entry 0 and advance
// by the *_bstride members (in words / scale elements / tensor elements).
struct QmvMat {
  const uint32_t* w;   // codes [n][k] (flat index row*k + col)
  const void* s;       // scales
  const uint32_t* w2;  // SwiGLU "up" partner, same shape (or null)
  const void* s2;
  const void* x;       // activations [m][x_rstride]
  void* y;             // outputs [m][y_rstride]
  const void* res;     // residual [m][r_rstride] (dtype of y) or null
  long long w_bstride, s_bstride, x_bstride, y_bstride, r_bstride;
  long long y_rstride; // elements between output rows of this matrix (row-major outputs)
  int y_hd;            // head dim of an attention head-packed output; 0: row-major
  int n;               // logical rows (output width N)
  int n_store;         // rows written: n plus zero-filled storage padding
  int tiles;           // row tiles per batch entry
  int tile_base;       // first workgroup of this matrix in the grid
  long long sk_off;    // split K: this matrix's first float in a partial plane
};

struct QmvParams {
  QmvMat mat[kMaxGroup];
  int nmat;
  int batch;
  int k;               // reduction length (shared)
  int m;               // activation rows
  int m_base;          // first activation row of this launch (row index of bias C)
  int y_rows;          // rows of a head-packed output tensor (its slices' row count)
  int group;           // scale block (elements); == k for per-row
  int groups_per_row;  // k / group
  int chunks;          // 16-byte code chunks per row
  int total_tiles;     // wave tiles over all matrices and batch entries
  long long x_rstride, r_rstride;  // elements between activation / residual rows
  float alpha, beta;
  const float* c;      // bias (C)
  int bcast;           // -1 none, 0 scalar, 1 per row m, 3 [m][n], 4 per column
  int c_rstride;       // elements between rows of C for bcast 3 (== n)
  const float* gamma;
  int gamma_size;
  float eps;
  int flags;
  // argmax partials (LM head): workgroups per row
  int parts;
  // in-kernel argmax merge (am_tagged non-null for every argmax launch).
  // Every workgroup stores its partial of row r
  // as three tagged words, tag << 32 | bits of (best, index, second), at
  // am_tagged[plane * am_plane + r * parts + workgroup]; the tag is the
  // launch's epoch, am_epoch[0] + 1 (0 skipped), read by every workgroup at
  // its start.  The last workgroup of the grid polls the words until all
  // carry the tag, merges them, writes the index / top-2 gap per row and
  // stores the tag back into am_epoch[0].  With am_group = g > 0 the merge
  // has two levels: the last workgroup of each full run of G = 2^g (index % G ==
  // G - 1, the grid's last excepted), groups = (grid - 1) / G runs, merges
  // its run into a group partial at r * parts + grid + run (parts = grid +
  // groups), and the grid's last workgroup merges its own run's partials and
  // the group partials, one contiguous range of each row.
  unsigned long long* am_tagged;
  long long am_plane;
  int am_group;
  unsigned* am_epoch;
  int32_t* am_out;
  float* am_gap;
  // split K (MFMA kernels): the K steps of every tile run as sk_chunks chunks
  // of sk_cs steps whose fp32 partials go to plane c of sk_part (plane c at
  // c * sk_plane floats; element (b, row, h, n) of matrix j at sk_off +
  // ((b * m + row) * NW + h) * n_store + n, h = 1 the SwiGLU up half);
  // splitk_reduce_launch sums them and applies the epilogue.  sk_chunks <= 1:
  // no split, the kernels finish their tiles themselves.
  float* sk_part;
  long long sk_plane;
  int sk_chunks;
  int sk_cs;
};

// The in-kernel argmax merge: at most kArgMergeRows activation rows per
// launch, the epoch word on a 256-byte line of its own (kArgEpochInts), and
// the merging workgroup's bounded wait for each partial (polls with a pause
// between them; about a second in all).
constexpr int kArgMergeRows = 32;
constexpr int kArgEpochInts = 64;
constexpr int kArgSpinLimit = 1 << 20;

// Streaming kernel registry (instantiated in aexq_qmv_q8.hip / aexq_qmv_q4.hip).
struct QmvConfig {
  int fmt, lpr, cpl, u, mmax;
  bool pair, argmax;
  int gmode;
};
typedef void (*QmvFn)(const QmvParams);
struct QmvEntry {
  QmvConfig cfg;
  QmvFn fn;
  int rw;  // rows per wave tile
};
const QmvEntry* qmv_table_q8(int* count);
const QmvEntry* qmv_table_q4(int* count);
const QmvEntry* qmv_find(const QmvConfig& cfg);
// resident workgroups of an entry per CU (occupancy query, cached)
int qmv_blocks_per_cu(const QmvEntry* e);
// Longest activation row a streaming launch stages in LDS (kFlagXShared):
// two passes of 8 elements per thread of a 256-thread workgroup.
constexpr int kQmvStageMaxK = 2 * kThreads * 8;
// Dynamic LDS of a streaming launch with kFlagXShared: the fp16 activation row
// and one fp32 partial per wave.
inline size_t qmv_stage_bytes(int k) { return (((size_t)k * 2 + 15) & ~(size_t)15) + kWaves * 4; }
hipError_t qmv_launch(const QmvEntry* e, const QmvParams& p, int grid, hipStream_t stream);

// Small-M MFMA kernel registry (aexq_qmm.hip): rows M <= 64 per launch.
struct QmmConfig {
  int fmt, gmode, mt, nt;
  bool pair, sf16;  // SwiGLU pair; fp16 (else fp32) scales
  bool wide;        // 256-wide K steps (aexq_qmmw.hpp; K % 256 == 0, Q8 or Q4 group 32)
  bool argmax;      // fused argmax partials (wide kernel only)
  bool rmsx;        // RMSNorm-in inside the kernel (wide kernel, one item per workgroup)
};
struct QmmEntry {
  QmmConfig cfg;
  QmvFn fn;
  int tn;  // weight rows per tile
};
const QmmEntry* qmm_find(const QmmConfig& cfg);
const QmmEntry* qmmw_table(int* count);  // the wide-step entries (aexq_qmmw.hip)
int qmm_blocks_per_cu(const QmmEntry* e);
hipError_t qmm_launch(const QmmEntry* e, const QmvParams& p, int grid, hipStream_t stream);
// Tiled GEMM for M > 32 rows (aexq_qgemm.hip): K % 64 == 0, Q8 or Q4 with a
// scale group of 16 or a multiple of 32, fp16 activation rows 16-byte aligned.
// Tiles are 128 weight rows (64 output columns for a SwiGLU pair) by bm rows.
struct QgemmConfig {
  int fmt, bm;
  bool pair, sf16;
  bool g16;    // Q4 with one scale per 16 codes
  bool direct; // LDS-direct pipeline (Q8; Q4 split scales in groups of 16 or 32)
  bool fd;     // Q4 weight tiles dequantised to fp16 (fp16(q * s)) for the MFMA
  bool k128;   // fd at 64-row tiles: 128-wide K steps (K a multiple of 128)
};
typedef void (*QgemmFn)(const QmvParams, int);
struct QgemmEntry {
  QgemmConfig cfg;
  QgemmFn fn;
};
const QgemmEntry* qgemm_find(const QgemmConfig& cfg);
int qgemm_rows_per_tile(bool pair);
int qgemm_blocks_per_cu(const QgemmEntry* e);
hipError_t qgemm_launch(const QgemmEntry* e, const QmvParams& p, hipStream_t stream);
// RMSNorm of activation rows into fp16 rows (the M > 1 form of RMSNorm-in):
// out[b][m][k] = fp16(x * rsqrt(max(mean(x^2) + eps, 1e-20)) * gamma[min(k, size-1)])
hipError_t rmsnorm_rows_launch(const void* x, int x_f32, long long x_rstride, long long x_bstride,
                               int batch, int m, int k, const float* gamma, int gamma_size,
                               float eps, void* out, hipStream_t stream);
hipError_t generic_launch(int fmt, const QmvParams& p, int grid, hipStream_t stream);
// Split-K fix-up of an MFMA launch (aexq_kernels.hip): for every output the
// sk_chunks partials summed in chunk order, then the epilogue of the MFMA
// kernels' finish(): Q8 row scale (q8_scale), bias / alpha / beta, SwiGLU
// (nw == 2), residual, the output layout.
hipError_t splitk_reduce_launch(const QmvParams& p, int nw, int q8_scale, int sf16,
                                hipStream_t stream);
int generic_rows_per_wg();
// element type of the logits an argmax pass reads
enum : int { kLogitsF32 = 0, kLogitsF16 = 1, kLogitsF32AsF16 = 2 };
// Argmax of p.m logits rows (row r at logits + r * rstride elements, n
// columns) in one launch of p.parts workgroups per row, `cols` columns each,
// merged in the launch through p's tagged partials into p.am_out / p.am_gap.
// vec > 1: 16-byte loads (logits, rstride and cols 16-byte aligned).
hipError_t logits_argmax_launch(const void* logits, int mode, int n, long long rstride, int cols,
                                int vec, const QmvParams& p, hipStream_t stream);
// The largest |scale| of `count` scales (fp16 or fp32) as fp32 bits, atomically
// maxed into *out (which the caller zeroes).
hipError_t scale_absmax_launch(const void* scales, long long count, int f16, unsigned* out,
                               hipStream_t stream);
// AQSGET8 Q8 / Q4 record payload (after its 24-byte header) into the device
// codes and fp32 scales of a weight with `count` elements.
hipError_t record_repack_launch(const void* payload, long long count, int block, int bits,
                                uint32_t* codes, float* scales, hipStream_t stream);
// Attention head-packed activation [b][ceil(heads/4)][rows][head_dim][4] ->
// dense rows [b][rows][heads*head_dim] of the same dtype (MM:1320-1389 reads).
hipError_t head_gather_launch(const void* src, int f32, int rows, int heads, int head_dim,
                              int batch, long long src_bstride, void* dst, hipStream_t stream);
hipError_t dequant_launch(int fmt, const uint32_t* w, const void* s, int scale_f16, int n, int k,
                          int group, float* out, hipStream_t stream);
hipError_t replicate_launch(const void* src, void* dst, long long bytes, int copies,
                            hipStream_t stream);

// decode-step kernels (aexq_decode.hip)
hipError_t embed_q8_launch(const uint32_t* codes, const void* scales, int scale_f16, int k,
                           const int32_t* tokens, int m, int vocab, void* out, hipStream_t stream);
hipError_t rope_kv_launch(void* q, const void* k, const void* v, void* kcache, void* vcache,
                          int hq, int hkv, int d, int cap, int pos, const float* cosv,
                          const float* sinv, hipStream_t stream);
// splits of a decode attention over `len` positions, and the most one launch takes
int attn_splits(int len);
int attn_max_splits();
int attn_part_stride();  // fp32 words per (head, split) partial row
int attn_counter_stride();  // ints between the kv heads' split counters
// part: hq * splits * (128 + 2) floats; counters: hkv ints, zero before the
// first launch (every launch leaves them zero).  knew/vnew/cosv/sinv non-null:
// RoPE of q and of the new k row plus the K/V append at position len - 1.
// posp non-null: the position is *posp (clamped to the capacity), read on the
// device, the grid is sized for `cap` positions and cosv/sinv are [cap][64]
// tables whose row *posp is used; `len` is ignored.
hipError_t attn_decode_launch(const void* q, const void* kcache, const void* vcache, int hq,
                              int hkv, int cap, int len, float scale, float* part, int* counters,
                              void* out, const void* knew, const void* vnew, const float* cosv,
                              const float* sinv, const int* posp, hipStream_t stream);
// One decode step's bookkeeping on the device: tokens_out[*position] (when
// non-null and the position is below out_cap) and *token take *argmax, then
// *position advances by one.
hipError_t decode_advance_launch(int* position, int* token, const int* argmax, int* tokens_out,
                                 int out_cap, hipStream_t stream);

}  // namespace aexq
