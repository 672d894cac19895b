/*
 * aexq_oracle.h -- CPU restatement of the Aexis quantized decode-linear path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * implementation in aiimage_amd/.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product path never does.
 *
 * Every function restates one piece of the reference (newzjh/AIImage, the
 * "Aexis" Unity engine, C#/HLSL).  Paths are relative to the reference root:
 *   GS  = Packages/com.aexis/Runtime/Execution/Graph/AexisGraphSession.cs
 *   Q8A = Packages/com.aexis/Runtime/Ncnn/NcnnCompute/NcnnQ8Archive.cs
 *   MM  = Packages/com.aexis/Runtime/Resources/Aexis/Includes/KernelGroups/AexisKernels.Pack4Matmul.hlsl
 *   CC  = Packages/com.aexis/Runtime/Resources/Aexis/AexisCommon.compute
 *   SP  = Packages/com.aexis/Runtime/Resources/Aexis/Includes/KernelGroups/AexisKernels.Pack4Spatial.hlsl
 *   DEC = Packages/com.aexis/Samples/AIImageApplicationExample/Runtime/Scripts/Qwen35DecoderSession.cs
 *   PN  = Packages/com.aexis/Runtime/Resources/Aexis/Includes/KernelGroups/AexisKernels.Pack4PointwiseNorm.hlsl
 */
#ifndef AEXQ_ORACLE_H
#define AEXQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* scale dtypes and nibble codes use the same numbering as include/aexq.h */
#define ORC_SCALE_F16 1
#define ORC_SCALE_F32 2
#define ORC_NIBBLE_TWOS 0    /* reference: q & 0xF, decode raw>=8 ? raw-16 : raw */
#define ORC_NIBBLE_OFFSET8 1 /* synthetic: q + 8, decode raw - 8 */

/* ---- scalar helpers ---------------------------------------------------- */
float orc_half_to_float(uint16_t h);
uint16_t orc_float_to_half(float f); /* IEEE binary16, round to nearest even */
int orc_round_to_int(float v);       /* Unity Mathf.RoundToInt (ties to even) */

/* ---- weight packers (load-time quantizers) ------------------------------ */
int orc_q8_pack_rows(const float* data, int rows, int cols, int contiguous,
                     uint32_t* packed, float* scales);
int orc_q4_pack_rows(const float* data, int rows, int cols, int contiguous,
                     uint32_t* packed, float* scales, int* scale_block);

/* ---- AQSGET8 archive records ------------------------------------------- */
#define ORC_RECORD_Q8 1
#define ORC_RECORD_RAW 2
#define ORC_RECORD_Q4 3
size_t orc_archive_header(uint8_t* out, int quant_bits, int default_block,
                          int record_count, int64_t source_bytes);
size_t orc_record_write_q8(const float* v, int n, int block, uint8_t* out);
size_t orc_record_write_q4(const float* v, int n, int block, uint8_t* out);
size_t orc_record_write_raw_f32(const float* v, int n, uint8_t* out);
size_t orc_record_write_q4_from_q8_rows(const uint32_t* q8_packed,
                                        const float* q8_scales, int rows,
                                        int row_size, int group, uint8_t* out);
int orc_archive_parse_header(const uint8_t* buf, size_t len, int* quant_bits,
                             int* default_block, int* record_count);
int orc_record_read_array(const uint8_t* rec, size_t len, int expected_count,
                          float* out, size_t* consumed);
int orc_record_read_q8_packed(const uint8_t* rec, size_t len, int expected_count,
                              int expected_block, uint32_t* packed, float* scales,
                              int* block, size_t* consumed);
int orc_record_read_q4_packed(const uint8_t* rec, size_t len, int expected_count,
                              int expected_block, uint32_t* packed, float* scales,
                              int* block, size_t* consumed);

/* ---- dequantize (the bit-exact target) ---------------------------------- */
int orc_dequant_q8(const uint32_t* words, const void* scales, int scale_dtype,
                   int n, int k, int block, float* out);
int orc_dequant_q4(const uint32_t* words, const void* scales, int scale_dtype,
                   int n, int k, int block, int nibble_code, float* out);

/* ---- Gemm ------------------------------------------------------------ */
void orc_gemm_cpu(const float* a, int m, int k, const float* b, int n,
                  int trans_b, float alpha, float beta, const float* c,
                  int broadcast_c, float* out);
void orc_gemm_cpu_mt(const float* a, int m, int k, const float* b, int n,
                     int trans_b, float alpha, float beta, const float* c,
                     int broadcast_c, float* out, int threads);
void orc_gemm_gpu_semantics(const float* a, int m, int k, const float* b, int n,
                            float alpha, float beta, const float* c,
                            int broadcast_c, double* out);

/* ---- epilogues --------------------------------------------------------- */
void orc_rmsnorm(const float* x, int rows, int width, float eps,
                 const float* gamma, int gamma_size, float* out);
float orc_swish(float x);
void orc_swiglu(const float* gate, const float* up, int n, float* out);

/* ---- LM head argmax ---------------------------------------------------- */
void orc_argmax_rows(const float* logits, int rows, int width, int64_t row_stride,
                     int32_t* out_index);

/* ---- decode step around the linears ------------------------------------ */
void orc_rope_table(int position, int head_dim, double base, float* cos_out, float* sin_out);
void orc_rope_rotate_half(const float* x, int heads, int head_dim, const float* cos_t,
                          const float* sin_t, float* out);
void orc_sdpa_decode(const float* q, const float* k, const float* v, int heads_q, int heads_kv,
                     int head_dim, int length, float scale, double* out);
/* attention head-packed layout (MM:1192-1389): [ceil(heads/4)][rows][head_dim][4] */
void orc_head_pack(const float* src, int rows, int heads, int head_dim, float* dst);
void orc_head_unpack(const float* src, int rows, int heads, int head_dim, float* dst);

#ifdef __cplusplus
}
#endif
#endif
