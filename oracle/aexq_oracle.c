/*
 * aexq_oracle.c -- CPU restatement of the Aexis quantized decode-linear path.
 *
 * TEST INFRASTRUCTURE ONLY (the parity checker and the CPU baseline).  The
 * product library in aiimage_amd/ never links or calls this file.
 *
 * Each function names the reference lines it restates (aliases are expanded
 * in aexq_oracle.h).  Arithmetic follows the reference's float32 order where
 * the reference defines the result bit for bit (packers, archive readers,
 * dequantization, argmax); the Gemm/RMSNorm/SwiGLU references accumulate in
 * float64 so they sit below the float32 noise of any GPU implementation.
 */
#include "aexq_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------------- */
/* scalar helpers                                                          */
/* ---------------------------------------------------------------------- */

static float bits_to_float(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static uint32_t float_to_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* IEEE binary16 -> binary32, exact (subnormals preserved). */
float orc_half_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t exp = (h >> 10) & 0x1f;
  uint32_t man = h & 0x3ff;
  if (exp == 0) {
    /* zero or subnormal: value = man * 2^-24, exact in float32 */
    float v = (float)man * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  if (exp == 31) return bits_to_float(sign | 0x7f800000u | (man << 13));
  return bits_to_float(sign | ((exp + 112) << 23) | (man << 13));
}

/* binary32 -> binary16, round to nearest even, with overflow to inf. */
uint16_t orc_float_to_half(float f) {
  uint32_t u = float_to_bits(f);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  uint32_t absu = u & 0x7fffffffu;
  if (absu >= 0x7f800000u) { /* inf or nan */
    if (absu > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((absu >> 13) & 0x3ffu));
    return (uint16_t)(sign | 0x7c00u);
  }
  if (absu >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to inf */
  if (absu < 0x38800000u) {
    /* result is subnormal or zero: scale to units of 2^-24 and round */
    double v = (double)bits_to_float(absu) * 16777216.0; /* exact */
    double r = nearbyint(v);                            /* ties to even */
    return (uint16_t)(sign | (uint16_t)r);
  }
  uint32_t exp = (absu >> 23) - 112;
  uint32_t man = absu & 0x7fffffu;
  uint32_t half = (exp << 10) | (man >> 13);
  uint32_t rest = man & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (half & 1u))) half += 1u;
  return (uint16_t)(sign | half);
}

/*
 * Unity Mathf.RoundToInt(f) == (int)Math.Round((double)f): ties to even.
 * The x64 CLR turns NaN and out-of-range doubles into int.MinValue; the
 * packers then clamp that to -127 / -7.
 */
int orc_round_to_int(float v) {
  double r = nearbyint((double)v);
  if (isnan(r) || r >= 2147483648.0 || r < -2147483648.0) return INT32_MIN;
  return (int)r;
}

/* Unity Mathf.Max(a, b) == a > b ? a : b (NaN handling follows from it). */
static float unity_max(float a, float b) { return a > b ? a : b; }
static int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* ---------------------------------------------------------------------- */
/* load-time packers                                                       */
/* ---------------------------------------------------------------------- */

/*
 * GS:12838-12885 NewInt8WeightOnlyUpload(float[] data, outputChannels,
 * valuesPerOutputChannel, outputChannelsAreContiguous): per output channel
 * scale = maxAbs/127 (1 when the channel is all zero), q = clamp(RoundToInt(
 * v/scale), -127, 127), byte (sourceIndex & 3) of word (sourceIndex >> 2).
 * `packed` must hold max(1, (rows*cols+3)/4) words; it is cleared here.
 */
int orc_q8_pack_rows(const float* data, int rows, int cols, int contiguous,
                     uint32_t* packed, float* scales) {
  if (!data || !packed || !scales || rows <= 0 || cols <= 0) return -1;
  size_t count = (size_t)rows * (size_t)cols;
  size_t words = count ? (count + 3) / 4 : 1;
  memset(packed, 0, words * sizeof(uint32_t));
  for (int oc = 0; oc < rows; ++oc) {
    float max_abs = 0.0f;
    for (int vi = 0; vi < cols; ++vi) {
      size_t src = contiguous ? (size_t)oc * cols + vi : (size_t)vi * rows + oc;
      max_abs = unity_max(max_abs, fabsf(data[src]));
    }
    float scale = max_abs > 0.0f ? max_abs / 127.0f : 1.0f;
    scales[oc] = scale;
    for (int vi = 0; vi < cols; ++vi) {
      size_t src = contiguous ? (size_t)oc * cols + vi : (size_t)vi * rows + oc;
      int q = clampi(orc_round_to_int(data[src] / scale), -127, 127);
      packed[src >> 2] |= (uint32_t)(uint8_t)(int8_t)q << ((src & 3) * 8);
    }
  }
  return 0;
}

/*
 * GS:12912-12964 NewInt4WeightOnlyUpload(float[] ...): per output channel
 * scale = maxAbs/7, q = clamp(RoundToInt(v/scale), -7, 7), nibble
 * (sourceIndex & 7) of word (sourceIndex >> 3), two's complement (q & 0xF).
 * scaleBlockSize = cols when channels are contiguous, else 0 (index by col).
 */
int orc_q4_pack_rows(const float* data, int rows, int cols, int contiguous,
                     uint32_t* packed, float* scales, int* scale_block) {
  if (!data || !packed || !scales || rows <= 0 || cols <= 0) return -1;
  size_t count = (size_t)rows * (size_t)cols;
  size_t words = count ? (count + 7) / 8 : 1;
  memset(packed, 0, words * sizeof(uint32_t));
  for (int oc = 0; oc < rows; ++oc) {
    float max_abs = 0.0f;
    for (int vi = 0; vi < cols; ++vi) {
      size_t src = contiguous ? (size_t)oc * cols + vi : (size_t)vi * rows + oc;
      max_abs = unity_max(max_abs, fabsf(data[src]));
    }
    float scale = max_abs > 0.0f ? max_abs / 7.0f : 1.0f;
    scales[oc] = scale;
    for (int vi = 0; vi < cols; ++vi) {
      size_t src = contiguous ? (size_t)oc * cols + vi : (size_t)vi * rows + oc;
      int q = clampi(orc_round_to_int(data[src] / scale), -7, 7);
      packed[src >> 3] |= ((uint32_t)q & 0xfu) << ((src & 7) * 4);
    }
  }
  if (scale_block) *scale_block = contiguous ? cols : 0;
  return 0;
}

/* ---------------------------------------------------------------------- */
/* AQSGET8 archive                                                         */
/* ---------------------------------------------------------------------- */

#define ORC_MAGIC 0x0038544547535141ULL /* Q8A:26 */
#define ORC_VERSION 1u                   /* Q8A:27 */
#define ORC_RECORD_MAGIC 0x31523851u     /* Q8A:28 "Q8R1" */

static void put_u32(uint8_t* p, uint32_t v) { memcpy(p, &v, 4); }
static void put_u64(uint8_t* p, uint64_t v) { memcpy(p, &v, 8); }
static uint32_t get_u32(const uint8_t* p) { uint32_t v; memcpy(&v, p, 4); return v; }
static uint64_t get_u64(const uint8_t* p) { uint64_t v; memcpy(&v, p, 8); return v; }

/* Q8A:60-65 archive header: magic, version, bits, default block, records, source bytes. */
size_t orc_archive_header(uint8_t* out, int quant_bits, int default_block,
                          int record_count, int64_t source_bytes) {
  if (out) {
    put_u64(out, ORC_MAGIC);
    put_u32(out + 8, ORC_VERSION);
    put_u32(out + 12, (uint32_t)quant_bits);
    put_u32(out + 16, (uint32_t)default_block);
    put_u32(out + 20, (uint32_t)record_count);
    put_u64(out + 24, (uint64_t)source_bytes);
  }
  return 32;
}

/* Q8A:236-245 record header (24 bytes). */
static size_t record_header(uint8_t* out, int kind, int count, int block, int payload) {
  if (out) {
    put_u32(out, ORC_RECORD_MAGIC);
    put_u32(out + 4, (uint32_t)kind);
    put_u32(out + 8, (uint32_t)count);
    put_u32(out + 12, (uint32_t)block);
    put_u32(out + 16, (uint32_t)payload);
    put_u32(out + 20, 0);
  }
  return 24;
}

static int block_count(int count, int block) { return count == 0 ? 0 : (count + block - 1) / block; }

/* Q8A:249-255 */
static int q4_payload_bytes(int count, int block) {
  int bytes = 0;
  for (int off = 0; off < count; off += block) {
    int len = block < count - off ? block : count - off;
    bytes += 4 + (len + 1) / 2;
  }
  return bytes;
}

/* Q8A:94-114 WriteQ8: per block a float32 scale (maxAbs/127) then int8 codes. */
size_t orc_record_write_q8(const float* v, int n, int block, uint8_t* out) {
  if (block <= 0 || n < 0) return 0;
  int payload = n + block_count(n, block) * 4;
  size_t pos = record_header(out, ORC_RECORD_Q8, n, block, payload);
  for (int off = 0; off < n; off += block) {
    int len = block < n - off ? block : n - off;
    float max_abs = 0.0f;
    for (int i = 0; i < len; ++i) max_abs = unity_max(max_abs, fabsf(v[off + i]));
    float scale = max_abs > 0.0f ? max_abs / 127.0f : 1.0f;
    if (out) memcpy(out + pos, &scale, 4);
    pos += 4;
    for (int i = 0; i < len; ++i) {
      int q = clampi(orc_round_to_int(v[off + i] / scale), -127, 127);
      if (out) out[pos] = (uint8_t)(int8_t)q;
      pos += 1;
    }
  }
  return pos;
}

/* Q8A:116-139 WriteQ4: per block a float32 scale (maxAbs/7) then nibbles, low nibble = even index. */
size_t orc_record_write_q4(const float* v, int n, int block, uint8_t* out) {
  if (block <= 0 || n < 0) return 0;
  size_t pos = record_header(out, ORC_RECORD_Q4, n, block, q4_payload_bytes(n, block));
  for (int off = 0; off < n; off += block) {
    int len = block < n - off ? block : n - off;
    float max_abs = 0.0f;
    for (int i = 0; i < len; ++i) max_abs = unity_max(max_abs, fabsf(v[off + i]));
    float scale = max_abs > 0.0f ? max_abs / 7.0f : 1.0f;
    if (out) memcpy(out + pos, &scale, 4);
    pos += 4;
    size_t nbytes = (size_t)(unsigned)(len + 1) / 2;
    if (out) memset(out + pos, 0, nbytes);
    for (int i = 0; i < len; ++i) {
      int q = clampi(orc_round_to_int(v[off + i] / scale), -7, 7);
      if (out) out[pos + (i >> 1)] |= (uint8_t)(((uint32_t)q & 0xfu) << ((i & 1) * 4));
    }
    pos += nbytes;
  }
  return pos;
}

/* Q8A:216-223 WriteFloat32Array: a raw record, block 1. */
size_t orc_record_write_raw_f32(const float* v, int n, uint8_t* out) {
  size_t pos = record_header(out, ORC_RECORD_RAW, n, 1, n * 4);
  if (out && n > 0) memcpy(out + pos, v, (size_t)n * 4);
  return pos + (size_t)n * 4;
}

/*
 * Q8A:167-207 WriteQ4FromQ8Rows: the shipping Q8 -> Q4 (group 16) conversion.
 * Per group: maxAbs over the int8 codes; scale = rowScale * maxAbs / 7;
 * q4 = clamp(RoundToInt(q8 * 7 / maxAbs), -7, 7).
 */
size_t orc_record_write_q4_from_q8_rows(const uint32_t* q8_packed,
                                        const float* q8_scales, int rows,
                                        int row_size, int group, uint8_t* out) {
  if (rows <= 0 || row_size <= 0 || group <= 0 || row_size % group != 0) return 0;
  int count = rows * row_size;
  size_t pos = record_header(out, ORC_RECORD_Q4, count, group, q4_payload_bytes(count, group));
  int gbytes = (group + 1) / 2;
  for (int row = 0; row < rows; ++row) {
    int row_start = row * row_size;
    for (int gs = 0; gs < row_size; gs += group) {
      int max_abs = 0;
      for (int c = 0; c < group; ++c) {
        int idx = row_start + gs + c;
        int8_t v = (int8_t)((q8_packed[idx >> 2] >> ((idx & 3) * 8)) & 0xffu);
        int a = v < 0 ? -(int)v : (int)v;
        if (a > max_abs) max_abs = a;
      }
      float scale = max_abs > 0 ? q8_scales[row] * (float)max_abs / 7.0f : 1.0f;
      if (out) memcpy(out + pos, &scale, 4);
      pos += 4;
      if (out) memset(out + pos, 0, (size_t)gbytes);
      for (int c = 0; c < group; ++c) {
        int idx = row_start + gs + c;
        int8_t q8 = (int8_t)((q8_packed[idx >> 2] >> ((idx & 3) * 8)) & 0xffu);
        int q4 = max_abs > 0 ? clampi(orc_round_to_int((float)q8 * 7.0f / (float)max_abs), -7, 7) : 0;
        if (out) out[pos + (c >> 1)] |= (uint8_t)(((uint32_t)q4 & 0xfu) << ((c & 1) * 4));
      }
      pos += (size_t)gbytes;
    }
  }
  return pos;
}

/* Q8A:277-291 archive header validation. Returns 0 or a negative error. */
int orc_archive_parse_header(const uint8_t* buf, size_t len, int* quant_bits,
                             int* default_block, int* record_count) {
  if (!buf || len < 32) return -1;
  if (get_u64(buf) != ORC_MAGIC) return -2;
  if (get_u32(buf + 8) != ORC_VERSION) return -3;
  int bits = (int)get_u32(buf + 12);
  int block = (int)get_u32(buf + 16);
  int records = (int)get_u32(buf + 20);
  if (block <= 0 || records < 0 || (bits != 0 && bits != 4 && bits != 8)) return -4;
  if (quant_bits) *quant_bits = bits == 0 ? 8 : bits; /* Q8A:293 */
  if (default_block) *default_block = block;
  if (record_count) *record_count = records;
  return 0;
}

/* Q8A:445-463 ReadHeader (element count must match; block > 0; payload >= 0). */
static int read_record_header(const uint8_t* rec, size_t len, int expected_count,
                              int* kind, int* block, int* payload) {
  if (!rec || len < 24) return -1;
  if (get_u32(rec) != ORC_RECORD_MAGIC) return -2;
  *kind = (int)get_u32(rec + 4);
  int count = (int)get_u32(rec + 8);
  *block = (int)get_u32(rec + 12);
  *payload = (int)get_u32(rec + 16);
  if (count != expected_count) return -3;
  if (*block <= 0 || *payload < 0) return -4;
  if (len < 24 + (size_t)*payload) return -5;
  return 0;
}

/*
 * Q8A:295-339 ReadArray: raw records are copied; Q8 records give
 * (sbyte)b * scale; Q4 records give (raw >= 8 ? raw - 16 : raw) * scale, both
 * in float32.  The payload size must match what was consumed (Q8A:465-469).
 */
int orc_record_read_array(const uint8_t* rec, size_t len, int expected_count,
                          float* out, size_t* consumed) {
  int kind, block, payload;
  int rc = read_record_header(rec, len, expected_count, &kind, &block, &payload);
  if (rc) return rc;
  const uint8_t* p = rec + 24;
  if (kind == ORC_RECORD_RAW) {
    if (payload != expected_count * 4) return -6;
    memcpy(out, p, (size_t)payload);
    if (consumed) *consumed = 24 + (size_t)payload;
    return 0;
  }
  if (kind != ORC_RECORD_Q8 && kind != ORC_RECORD_Q4) return -7;
  size_t used = 0;
  for (int off = 0; off < expected_count; off += block) {
    int blen = block < expected_count - off ? block : expected_count - off;
    if (used + 4 > (size_t)payload) return -8;
    float scale;
    memcpy(&scale, p + used, 4);
    used += 4;
    if (kind == ORC_RECORD_Q8) {
      if (used + (size_t)blen > (size_t)payload) return -8;
      for (int i = 0; i < blen; ++i) out[off + i] = (float)(int8_t)p[used + i] * scale;
      used += (size_t)blen;
    } else {
      int nbytes = (blen + 1) / 2;
      if (used + (size_t)nbytes > (size_t)payload) return -8;
      for (int i = 0; i < blen; ++i) {
        int raw = (p[used + (i >> 1)] >> ((i & 1) * 4)) & 0xf;
        int s = raw >= 8 ? raw - 16 : raw;
        out[off + i] = (float)s * scale;
      }
      used += (size_t)nbytes;
    }
  }
  if (used != (size_t)payload) return -9;
  if (consumed) *consumed = 24 + used;
  return 0;
}

/* Q8A:341-367 ReadPackedArray: int8 codes into uint32 words, lane (index & 3). */
int orc_record_read_q8_packed(const uint8_t* rec, size_t len, int expected_count,
                              int expected_block, uint32_t* packed, float* scales,
                              int* block_out, size_t* consumed) {
  int kind, block, payload;
  int rc = read_record_header(rec, len, expected_count, &kind, &block, &payload);
  if (rc) return rc;
  if (kind != ORC_RECORD_Q8) return -7;
  if (expected_block > 0 && block != expected_block) return -10;
  size_t words = expected_count ? ((size_t)expected_count + 3) / 4 : 1;
  memset(packed, 0, words * 4);
  const uint8_t* p = rec + 24;
  size_t used = 0;
  int nblocks = block_count(expected_count, block);
  for (int b = 0; b < nblocks; ++b) {
    int off = b * block;
    int blen = block < expected_count - off ? block : expected_count - off;
    if (used + 4 + (size_t)blen > (size_t)payload) return -8;
    memcpy(&scales[b], p + used, 4);
    used += 4;
    for (int i = 0; i < blen; ++i) {
      int idx = off + i;
      packed[idx >> 2] |= (uint32_t)p[used + i] << ((idx & 3) * 8);
    }
    used += (size_t)blen;
  }
  if (used != (size_t)payload) return -9;
  if (block_out) *block_out = block;
  if (consumed) *consumed = 24 + used;
  return 0;
}

/* Q8A:385-413 ReadQ4PackedArray: nibbles into uint32 words, lane (index & 7). */
int orc_record_read_q4_packed(const uint8_t* rec, size_t len, int expected_count,
                              int expected_block, uint32_t* packed, float* scales,
                              int* block_out, size_t* consumed) {
  int kind, block, payload;
  int rc = read_record_header(rec, len, expected_count, &kind, &block, &payload);
  if (rc) return rc;
  if (kind != ORC_RECORD_Q4) return -7;
  if (expected_block > 0 && block != expected_block) return -10;
  size_t words = expected_count ? ((size_t)expected_count + 7) / 8 : 1;
  memset(packed, 0, words * 4);
  const uint8_t* p = rec + 24;
  size_t used = 0;
  int nblocks = block_count(expected_count, block);
  for (int b = 0; b < nblocks; ++b) {
    int off = b * block;
    int blen = block < expected_count - off ? block : expected_count - off;
    int nbytes = (blen + 1) / 2;
    if (used + 4 + (size_t)nbytes > (size_t)payload) return -8;
    memcpy(&scales[b], p + used, 4);
    used += 4;
    for (int i = 0; i < blen; ++i) {
      int idx = off + i;
      uint32_t raw = (uint32_t)((p[used + (i >> 1)] >> ((i & 1) * 4)) & 0xf);
      packed[idx >> 3] |= raw << ((idx & 7) * 4);
    }
    used += (size_t)nbytes;
  }
  if (used != (size_t)payload) return -9;
  if (block_out) *block_out = block;
  if (consumed) *consumed = 24 + used;
  return 0;
}

/* ---------------------------------------------------------------------- */
/* dequantize                                                              */
/* ---------------------------------------------------------------------- */

static float read_scale(const void* scales, int dtype, size_t i) {
  if (dtype == ORC_SCALE_F16) return orc_half_to_float(((const uint16_t*)scales)[i]);
  return ((const float*)scales)[i];
}

/*
 * MM:722-727 AexisGemm2DReadB, INT8 branch with transB: index = col*K + kk,
 * raw = byte (index & 3) of word (index >> 2), signed = raw >= 128 ? raw-256 :
 * raw, w = float(signed) * scales[col].  The GPU path only admits one scale
 * per output row (GS:12893-12894), so `block` must be K (or 0 for "per row").
 * fp16 scales (the synthetic format) are widened exactly, subnormals kept.
 */
int orc_dequant_q8(const uint32_t* words, const void* scales, int scale_dtype,
                   int n, int k, int block, float* out) {
  if (!words || !scales || !out || n <= 0 || k <= 0) return -1;
  if (block != 0 && block != k) return -2;
  for (int col = 0; col < n; ++col) {
    float s = read_scale(scales, scale_dtype, (size_t)col);
    for (int kk = 0; kk < k; ++kk) {
      size_t idx = (size_t)col * k + kk;
      uint32_t raw = (words[idx >> 2] >> ((idx & 3) * 8)) & 0xffu;
      int sv = raw >= 128u ? (int)raw - 256 : (int)raw;
      out[idx] = (float)sv * s;
    }
  }
  return 0;
}

/*
 * MM:712-720 AexisGemm2DReadB, INT4 branch with transB: raw = nibble
 * (index & 7) of word (index >> 3); signed = raw >= 8 ? raw-16 : raw for the
 * reference's two's-complement code, raw - 8 for the offset-8 code;
 * scaleIndex = block > 0 ? index / block : col; w = float(signed) * scale.
 */
int orc_dequant_q4(const uint32_t* words, const void* scales, int scale_dtype,
                   int n, int k, int block, int nibble_code, float* out) {
  if (!words || !scales || !out || n <= 0 || k <= 0 || block < 0) return -1;
  for (int col = 0; col < n; ++col) {
    for (int kk = 0; kk < k; ++kk) {
      size_t idx = (size_t)col * k + kk;
      uint32_t raw = (words[idx >> 3] >> ((idx & 7) * 4)) & 0xfu;
      int sv = nibble_code == ORC_NIBBLE_OFFSET8 ? (int)raw - 8
                                                 : (raw >= 8u ? (int)raw - 16 : (int)raw);
      size_t si = block > 0 ? idx / (size_t)block : (size_t)col;
      out[idx] = (float)sv * read_scale(scales, scale_dtype, si);
    }
  }
  return 0;
}

/* ---------------------------------------------------------------------- */
/* Gemm                                                                    */
/* ---------------------------------------------------------------------- */

/* GS:13363-13373 broadcast of C. */
static float resolve_c(const float* c, int bcast, int row, int col, int n) {
  switch (bcast) {
    case 0: return c[0];
    case 1: return c[row];
    case 2: return c[row];
    case 3: return c[(size_t)row * n + col];
    case 4: return c[col];
    default: return 0.0f;
  }
}

static float gemm_cpu_cell(const float* a, int k, const float* b, int n, int trans_b,
                           float alpha, float beta, const float* c, int bcast,
                           int row, int col) {
  double sum = 0.0;
  const float* arow = a + (size_t)row * k;
  for (int kk = 0; kk < k; ++kk) {
    float bv = trans_b ? b[(size_t)col * k + kk] : b[(size_t)kk * n + col];
    sum += (double)arow[kk] * (double)bv;
  }
  float value = alpha * (float)sum;
  if (c && bcast != -1) value += beta * resolve_c(c, bcast, row, col, n);
  return value;
}

/*
 * GS:13328-13381 RunGemmCpu, the reference's CPU path: a single-threaded
 * triple loop, float64 accumulation of (double)a * (double)b, then
 * alpha * (float)sum + beta * C.  For quantized layers `b` is the float32
 * dequantized weight (Q8A:295-339 ReadArray or MM:707-727).
 */
void orc_gemm_cpu(const float* a, int m, int k, const float* b, int n,
                  int trans_b, float alpha, float beta, const float* c,
                  int broadcast_c, float* out) {
  for (int row = 0; row < m; ++row)
    for (int col = 0; col < n; ++col)
      out[(size_t)row * n + col] =
          gemm_cpu_cell(a, k, b, n, trans_b, alpha, beta, c, broadcast_c, row, col);
}

typedef struct {
  const float* a; const float* b; const float* c; float* out;
  int m, k, n, trans_b, bcast; float alpha, beta;
  int t, threads;
} gemm_job;

static void* gemm_worker(void* arg) {
  gemm_job* j = (gemm_job*)arg;
  size_t cells = (size_t)j->m * j->n;
  size_t lo = cells * j->t / j->threads, hi = cells * (j->t + 1) / j->threads;
  for (size_t i = lo; i < hi; ++i) {
    int row = (int)(i / j->n), col = (int)(i % j->n);
    j->out[i] = gemm_cpu_cell(j->a, j->k, j->b, j->n, j->trans_b, j->alpha, j->beta,
                              j->c, j->bcast, row, col);
  }
  return NULL;
}

/* RunGemmCpu split over output cells on `threads` host threads; each cell is
 * computed exactly as in the single-threaded loop, so results are identical. */
void orc_gemm_cpu_mt(const float* a, int m, int k, const float* b, int n,
                     int trans_b, float alpha, float beta, const float* c,
                     int broadcast_c, float* out, int threads) {
  if (threads <= 1) {
    orc_gemm_cpu(a, m, k, b, n, trans_b, alpha, beta, c, broadcast_c, out);
    return;
  }
  if (threads > 256) threads = 256;
  pthread_t tid[256];
  gemm_job jobs[256];
  for (int t = 0; t < threads; ++t) {
    gemm_job j = {a, b, c, out, m, k, n, trans_b, broadcast_c, alpha, beta, t, threads};
    jobs[t] = j;
    pthread_create(&tid[t], NULL, gemm_worker, &jobs[t]);
  }
  for (int t = 0; t < threads; ++t) pthread_join(tid[t], NULL);
}

/*
 * MM:1038-1104 / MM:1106-1190 (Pack4-linear Gemm) semantics with transB:
 * the accumulator starts at beta*C (MM:1054-1057, AexisResolveGemm2DBias
 * MM:688-705 with broadcast types 0/1/3/4), adds sum_k a*w, and the result is
 * scaled by alpha (MM:1101).  Accumulated in float64 as the parity reference.
 * b is [n][k] (transB).  c may be NULL (no C).
 */
void orc_gemm_gpu_semantics(const float* a, int m, int k, const float* b, int n,
                            float alpha, float beta, const float* c,
                            int broadcast_c, double* out) {
  for (int row = 0; row < m; ++row) {
    for (int col = 0; col < n; ++col) {
      double acc = 0.0;
      if (c && broadcast_c != 2 && broadcast_c >= 0 && broadcast_c <= 4)
        acc = (double)beta * (double)resolve_c(c, broadcast_c, row, col, n);
      const float* arow = a + (size_t)row * k;
      const float* brow = b + (size_t)col * k;
      for (int kk = 0; kk < k; ++kk) acc += (double)arow[kk] * (double)brow[kk];
      out[(size_t)row * n + col] = (double)alpha * acc;
    }
  }
}

/* ---------------------------------------------------------------------- */
/* epilogues                                                               */
/* ---------------------------------------------------------------------- */

/*
 * CC:4531-4557 AexisRmsNormPack4LinearMat: per row, invRms = rsqrt(max(
 * sum(x^2)/W + eps, 1e-20)); y = x * invRms * gamma[clamp(i, 0, size-1)].
 * gamma may be NULL (affine off).  float64 arithmetic.
 */
void orc_rmsnorm(const float* x, int rows, int width, float eps,
                 const float* gamma, int gamma_size, float* out) {
  int w = width > 0 ? width : 1;
  for (int r = 0; r < rows; ++r) {
    const float* xr = x + (size_t)r * width;
    double ss = 0.0;
    for (int i = 0; i < width; ++i) ss += (double)xr[i] * (double)xr[i];
    double ms = ss / (double)w + (double)eps;
    if (ms < 1e-20) ms = 1e-20;
    double inv = 1.0 / sqrt(ms);
    for (int i = 0; i < width; ++i) {
      double v = (double)xr[i] * inv;
      if (gamma && gamma_size > 0) v *= (double)gamma[clampi(i, 0, gamma_size - 1)];
      out[(size_t)r * width + i] = (float)v;
    }
  }
}

/* MM:106-116 AexisSwishPack4_Impl: y = x / (1 + exp(-x)), in float64. */
float orc_swish(float x) { return (float)((double)x / (1.0 + exp(-(double)x))); }

/* The SwiGLU-out pair: Swish(gate) (MM:106-116) then BinaryOp Mul with up
 * (SP:819-831), evaluated in float64 and rounded once. */
void orc_swiglu(const float* gate, const float* up, int n, float* out) {
  for (int i = 0; i < n; ++i) {
    double g = (double)gate[i];
    out[i] = (float)(g / (1.0 + exp(-g)) * (double)up[i]);
  }
}

/* ---------------------------------------------------------------------- */
/* argmax                                                                  */
/* ---------------------------------------------------------------------- */

/*
 * MM:645-686 AexisArgMaxPack4LinearMat_Impl (CPU twin DEC:1902-1908): scan
 * the logical width, take element 0, then any later element with
 * value > best.  The first maximum wins; NaN never replaces a value, and a
 * NaN at index 0 is never replaced.
 */
void orc_argmax_rows(const float* logits, int rows, int width, int64_t row_stride,
                     int32_t* out_index) {
  for (int r = 0; r < rows; ++r) {
    const float* row = logits + (size_t)r * (size_t)row_stride;
    int best_index = 0;
    float best_value = 0.0f;
    for (int i = 0; i < width; ++i) {
      float v = row[i];
      if (i == 0 || v > best_value) {
        best_value = v;
        best_index = i;
      }
    }
    out_index[r] = best_index;
  }
}

/* ---------------------------------------------------------------------- */
/* decode step around the linears                                          */
/* ---------------------------------------------------------------------- */

/*
 * DEC:1660-1675 CreateRopeTextures, the row of one position, in the float32
 * steps the C# evaluates: e = j * (2f / (half * 2f)); p = Mathf.Pow(theta, e);
 * inverse = 1f / p; angle = position * inverse (float multiply); entries
 * Mathf.Cos(angle), Mathf.Sin(angle).  UnityEngine's Mathf.Pow/Cos/Sin take
 * and return float and evaluate System.Math's double routines in between,
 * i.e. (float)pow((double)a, (double)b) and (float)cos((double)a).  theta is
 * the float constant RopeTheta (DEC:172), hence the cast of `base`.
 */
void orc_rope_table(int position, int head_dim, double base, float* cos_out, float* sin_out) {
  int half = head_dim / 2;
  float theta = (float)base;
  float step = 2.0f / ((float)half * 2.0f);
  for (int j = 0; j < half; ++j) {
    float e = (float)j * step;
    float p = (float)pow((double)theta, (double)e);
    float inverse = 1.0f / p;
    float angle = (float)position * inverse;
    cos_out[j] = (float)cos((double)angle);
    sin_out[j] = (float)sin((double)angle);
  }
}

/*
 * PN:414-473 AexisRotaryEmbedPack4_Impl, non-interleaved branch: for pair
 * (j, j + half): first = x0*cos - x1*sin, second = x0*sin + x1*cos, with the
 * table entry j of the position.  x and out are [heads][head_dim].
 */
void orc_rope_rotate_half(const float* x, int heads, int head_dim, const float* cos_t,
                          const float* sin_t, float* out) {
  int half = head_dim / 2;
  for (int h = 0; h < heads; ++h) {
    const float* r = x + (size_t)h * head_dim;
    float* o = out + (size_t)h * head_dim;
    for (int j = 0; j < half; ++j) {
      float x0 = r[j], x1 = r[j + half];
      o[j] = x0 * cos_t[j] - x1 * sin_t[j];
      o[j + half] = x0 * sin_t[j] + x1 * cos_t[j];
    }
  }
}

/*
 * MM:420-544 AexisSdpaAttentionPack4CDHW_Impl for one query row: query head h
 * reads key head h / (heads_q / heads_kv); s_j = (q . k_j) * scale; the
 * softmax subtracts the maximum and divides by max(sum, 1e-20); out = sum_j
 * p_j v_j.  Evaluated in float64.  q [heads_q][d], k/v [heads_kv][length][d].
 */
void orc_sdpa_decode(const float* q, const float* k, const float* v, int heads_q, int heads_kv,
                     int head_dim, int length, float scale, double* out) {
  int group = heads_q / heads_kv;
  if (group < 1) group = 1;
  double* s = (double*)malloc(sizeof(double) * (size_t)(length > 0 ? length : 1));
  for (int h = 0; h < heads_q; ++h) {
    int g = h / group;
    if (g > heads_kv - 1) g = heads_kv - 1;
    const float* qh = q + (size_t)h * head_dim;
    double mx = -1.0e300;
    for (int j = 0; j < length; ++j) {
      const float* kj = k + ((size_t)g * length + j) * head_dim;
      double acc = 0.0;
      for (int i = 0; i < head_dim; ++i) acc += (double)qh[i] * (double)kj[i];
      s[j] = acc * (double)scale;
      if (s[j] > mx) mx = s[j];
    }
    double sum = 0.0;
    for (int j = 0; j < length; ++j) {
      s[j] = exp(s[j] - mx);
      sum += s[j];
    }
    double inv = 1.0 / (sum > 1e-20 ? sum : 1e-20);
    for (int i = 0; i < head_dim; ++i) {
      double acc = 0.0;
      for (int j = 0; j < length; ++j)
        acc += s[j] * inv * (double)v[((size_t)g * length + j) * head_dim + i];
      out[(size_t)h * head_dim + i] = acc;
    }
  }
  free(s);
}

/*
 * Attention head-packed texture layout.  The Q/K/V Gemm variants write
 * _GemmTexOutArr[int3(dim, row, head / 4)] with lane head % 4 set by
 * AexisWriteLane and the lanes of heads past numHeads left 0
 * (MM:1192-1318); o_proj reads its input through
 * AexisReadPack4Channel(arr, dim, row, head) (MM:1320-1389).  Storage is
 * BufferShape {3, head_dim, rows, 1, heads} (GL:1003-1043): a texture array
 * of ceil(heads / 4) slices of rows x head_dim float4 texels, so element
 * (row, head * head_dim + d) of the logical [rows][heads * head_dim] matrix
 * sits at (((head / 4) * rows + row) * head_dim + d) * 4 + head % 4.
 * dst holds ceil(heads / 4) * rows * head_dim * 4 values.
 */
void orc_head_pack(const float* src, int rows, int heads, int head_dim, float* dst) {
  const size_t total = (size_t)((heads + 3) / 4) * rows * head_dim * 4;
  for (size_t i = 0; i < total; ++i) dst[i] = 0.0f;
  for (int r = 0; r < rows; ++r)
    for (int h = 0; h < heads; ++h)
      for (int d = 0; d < head_dim; ++d)
        dst[(((size_t)(h / 4) * rows + r) * head_dim + d) * 4 + (h % 4)] =
            src[(size_t)r * heads * head_dim + (size_t)h * head_dim + d];
}

void orc_head_unpack(const float* src, int rows, int heads, int head_dim, float* dst) {
  for (int r = 0; r < rows; ++r)
    for (int h = 0; h < heads; ++h)
      for (int d = 0; d < head_dim; ++d)
        dst[(size_t)r * heads * head_dim + (size_t)h * head_dim + d] =
            src[(((size_t)(h / 4) * rows + r) * head_dim + d) * 4 + (h % 4)];
}
