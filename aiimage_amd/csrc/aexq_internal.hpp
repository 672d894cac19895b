// Shared host/device definitions of the aexq HIP library (not part of the ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace aexq {

constexpr int kMaxGroup = 8;  // matrices per grouped launch
constexpr int kWaves = 4;     // waves per workgroup of the matvec kernels
constexpr int kThreads = 64 * kWaves;

enum Fmt : int { kQ8 = 0, kQ4 = 1 };

// Flags inside QmvParams::flags.
enum : int {
  kFlagRms = 1,        // RMSNorm-in prologue
  kFlagResidual = 2,   // y += residual
  kFlagYf32 = 4,       // output is fp32 (else fp16)
  kFlagAlphaIn = 8,    // alpha * (beta*C + sum) (Pack4 linear); else beta*C + alpha*sum (tiled)
  kFlagScaleF16 = 16,  // scales are fp16 (else fp32)
  kFlagXf32 = 32,      // activations fp32 (generic kernel only)
};

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
  long long y_rstride; // elements between output rows of this matrix
  int n;               // logical rows (output width N)
  int n_store;         // rows written: n plus zero-filled storage padding
  int tiles;           // row tiles per batch entry
  int tile_base;       // first workgroup of this matrix in the grid
};

struct QmvParams {
  QmvMat mat[kMaxGroup];
  int nmat;
  int batch;
  int k;               // reduction length (shared)
  int m;               // activation rows
  int group;           // scale block (elements); == k for per-row
  int groups_per_row;  // k / group
  int chunks;          // 16-byte code chunks per row
  uint32_t xor_mask;   // 0x88888888 turns two's-complement nibbles into offset-8
  long long x_rstride, r_rstride;  // elements between activation / residual rows
  float alpha, beta;
  const float* c;      // bias (C)
  int bcast;           // -1 none, 0 scalar, 1 per row m, 3 [m][n], 4 per column
  int c_rstride;       // elements between rows of C for bcast 3 (== n)
  const float* gamma;
  int gamma_size;
  float eps;
  int flags;
  // argmax partials (LM head): [m][parts]
  float* part_best;
  int* part_index;
  float* part_second;
  int parts;
};

struct ArgmaxParams {
  const float* pv;
  const int* pi;
  const float* ps;
  int parts;
  int m;
  int32_t* out_index;
  float* out_gap;
};

// host-side launchers (defined in aexq_qmv.hip)
struct QmvConfig {
  int fmt, lpr, cpl, mmax;
  bool pair, argmax, g16;
};
int qmv_rows_per_wg(const QmvConfig& cfg);
hipError_t qmv_launch(const QmvConfig& cfg, const QmvParams& p, int grid, hipStream_t stream);
bool qmv_has_config(const QmvConfig& cfg);
hipError_t generic_launch(int fmt, const QmvParams& p, int grid, hipStream_t stream);
int generic_rows_per_wg();
hipError_t argmax_finalize_launch(const ArgmaxParams& a, hipStream_t stream);
hipError_t logits_argmax_launch(const float* logits, int m, int n, long long rstride, float* pv,
                                int* pi, float* ps, int parts, hipStream_t stream);
int logits_argmax_cols_per_wg();
hipError_t dequant_launch(int fmt, const uint32_t* w, const void* s, int scale_f16, int n, int k,
                          int group, uint32_t xor_mask, float* out, hipStream_t stream);
hipError_t replicate_launch(const void* src, void* dst, long long bytes, int copies,
                            hipStream_t stream);

}  // namespace aexq
