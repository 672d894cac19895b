// C-ABI implementation of include/aexq.h: contexts, library-owned weights, the
// strict plan (kernel selection with diagnostics, never a fallback) and the
// launches.  Reference citations use the aliases listed in include/aexq.h.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>
#include <string>
#include <vector>

#include "../../include/aexq.h"
#include "aexq_internal.hpp"
#include "aexq_step.hpp"

using namespace aexq;

// ---------------------------------------------------------------------------
// errors
// ---------------------------------------------------------------------------
static thread_local std::string g_last_error;

static aexq_status fail(aexq_status st, const char* op, const char* fmt, ...) {
  char buf[768];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = std::string("aexq: ") + op + " failed | " + buf;
  return st;
}

static aexq_status hip_fail(hipError_t e, const char* op, const char* what) {
  return fail(e == hipErrorOutOfMemory ? AEXQ_ERR_OUT_OF_MEMORY : AEXQ_ERR_DEVICE, op,
              "%s | hip=%s", what, hipGetErrorString(e));
}

#define HIP_TRY(op, expr)                                   \
  do {                                                      \
    hipError_t _e = (expr);                                 \
    if (_e != hipSuccess) return hip_fail(_e, op, #expr);   \
  } while (0)

// ---------------------------------------------------------------------------
// objects
// ---------------------------------------------------------------------------
struct aexq_ctx {
  int device = 0;
  int cus = 256;  // compute units of the device
  hipStream_t stream = nullptr;
  // Scratch buffers, grown on demand (capacities in bytes).
  float* logits_scratch = nullptr;
  long long logits_cap = 0;
  // RMS-normalised activation rows of the MFMA path
  void* act_scratch = nullptr;
  long long act_cap = 0;
  void* gather_scratch = nullptr;  // dense rows of a head-packed x
  long long gather_cap = 0;
  // decode attention split partials
  float* attn_part = nullptr;
  long long attn_cap = 0;
  int* attn_count = nullptr;  // per kv head: splits finished in the running launch
  long long attn_count_cap = 0;
  // split-K partial planes of the MFMA kernels
  float* sk_part = nullptr;
  long long sk_cap = 0;
  // tagged argmax partials of the in-kernel merge (three planes) and its epoch
  // word (both zeroed at allocation)
  unsigned long long* am_tagged = nullptr;
  long long am_tagged_cap = 0;
  unsigned* am_epoch = nullptr;
  long long am_epoch_cap = 0;
  // scratch buffers replaced by larger ones: a HIP graph captured before the
  // growth still holds their addresses, so they live until aexq_destroy
  std::vector<void*> retired;
  // the device address of the no-allocation entry point's `scratch` array
  unsigned long long* noalloc = nullptr;
};

struct aexq_weight {
  // the device holding the buffers; a weight may outlive the context that
  // made it, so release never reaches back into the context
  int device = 0;
  int bits = 8;
  int n = 0, k = 0;
  int block = 0;        // scale block in flat elements (k for per-row)
  int scale_dtype = AEXQ_DTYPE_F32;
  int nibble_code = AEXQ_NIBBLE_TWOS;
  int batch = 1;
  uint32_t* codes = nullptr;
  void* scales = nullptr;
  long long code_bytes = 0;    // per copy, unpadded
  long long scale_count = 0;   // per copy
  long long code_stride = 0;   // bytes between copies
  long long scale_stride = 0;  // bytes between copies
  bool owns = true;
  // Q4: every scale's fp16(q * s) stays finite (8 |s| <= 65504), so the tiled
  // GEMM may dequantise weight tiles to fp16 (set once the scales are on the device)
  bool fp16_dequant_ok = false;
};

static long long round_up(long long v, long long a) { return (v + a - 1) / a * a; }

// ---------------------------------------------------------------------------
// Scratch of aexq_lmhead_argmax_noalloc: the tagged argmax partials of one
// launch (three planes of kNoAllocParts 64-bit words: best, index, second, one
// word per workgroup and activation row) and the epoch word, in a file-scope
// device array instead of memory the library allocates.  Each GPU holds its
// own copy from module load to process exit; its address on a device comes
// from hipGetSymbolAddress, taken once per device when the first context on
// that device is created.  The array is zero-initialised at load; every call
// tags its partials with the epoch plus one and leaves that tag as the next
// epoch, so no call clears anything.  Calls that overlap on one GPU (other
// streams or contexts) share the array and race.
// ---------------------------------------------------------------------------
constexpr long long kNoAllocParts = 16384;  // 3 x 128 KiB
static __device__ __align__(256) unsigned long long scratch[3 * kNoAllocParts + kArgEpochInts / 2];
constexpr int kMaxDevices = 64;
static std::mutex g_noalloc_mu;
static unsigned long long* g_noalloc_ptr[kMaxDevices];  // device address of `scratch` per device
static hipError_t g_noalloc_err[kMaxDevices];  // why it is missing, if it is

// With `device` current: the device address of `scratch` on it (once).
static unsigned long long* noalloc_scratch(int device) {
  if (device < 0 || device >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  if (!g_noalloc_ptr[device] && g_noalloc_err[device] == hipSuccess) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e == hipSuccess && p) {
      g_noalloc_ptr[device] = (unsigned long long*)p;
    } else {
      g_noalloc_err[device] = e != hipSuccess ? e : hipErrorInvalidSymbol;
      (void)hipGetLastError();  // leave no sticky error for the caller's next launch
    }
  }
  return g_noalloc_ptr[device];
}

// Makes the context scratch buffer *buf hold at least `bytes`.  A buffer that
// is replaced is retired, not freed (a HIP graph captured earlier may still
// hold its address), and growth while the context's stream is capturing is
// refused: hipMalloc cannot be recorded into a graph, so every scratch size a
// captured sequence needs is reached by running it once before the capture.
// `zero` clears a new buffer (the attention split counters start at zero).
static aexq_status grow_scratch(aexq_ctx* ctx, void** buf, long long* cap, long long bytes,
                                const char* op, const char* what, bool zero = false) {
  if (bytes <= *cap) return AEXQ_OK;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(ctx->stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
    return fail(AEXQ_ERR_UNSUPPORTED, op,
                "%s scratch must grow from %lld to %lld bytes while the stream is capturing | "
                "run the same calls once before the capture", what, *cap, bytes);
  void* nb = nullptr;
  hipError_t e = hipMalloc(&nb, (size_t)bytes);
  if (e == hipSuccess && zero) e = hipMemset(nb, 0, (size_t)bytes);
  if (e != hipSuccess) {
    (void)hipFree(nb);
    return hip_fail(e, op, what);
  }
  if (*buf) ctx->retired.push_back(*buf);
  *buf = nb;
  *cap = bytes;
  return AEXQ_OK;
}
static int scale_bytes(int dtype) { return dtype == AEXQ_DTYPE_F16 ? 2 : 4; }

extern "C" int aexq_abi_version(void) { return AEXQ_ABI_VERSION; }
extern "C" const char* aexq_last_error(void) { return g_last_error.c_str(); }

extern "C" aexq_status aexq_create(int device, void* hip_stream, aexq_ctx** out) {
  if (!out) return fail(AEXQ_ERR_INVALID_ARGUMENT, "aexq_create", "out is NULL");
  int count = 0;
  HIP_TRY("aexq_create", hipGetDeviceCount(&count));
  if (device < 0 || device >= count)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, "aexq_create", "device=%d of %d", device, count);
  HIP_TRY("aexq_create", hipSetDevice(device));
  int cus = 0;
  HIP_TRY("aexq_create", hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device));
  aexq_ctx* c = new aexq_ctx();
  c->device = device;
  c->cus = cus > 0 ? cus : 1;
  c->stream = (hipStream_t)hip_stream;
  c->noalloc = noalloc_scratch(device);  // null: aexq_lmhead_argmax_noalloc reports why
  *out = c;
  return AEXQ_OK;
}

extern "C" void aexq_destroy(aexq_ctx* ctx) {
  if (!ctx) return;
  (void)hipSetDevice(ctx->device);
  (void)hipFree(ctx->logits_scratch);
  (void)hipFree(ctx->act_scratch);
  (void)hipFree(ctx->gather_scratch);
  (void)hipFree(ctx->attn_part);
  (void)hipFree(ctx->attn_count);
  (void)hipFree(ctx->sk_part);
  (void)hipFree(ctx->am_tagged);
  (void)hipFree(ctx->am_epoch);
  for (void* b : ctx->retired) (void)hipFree(b);
  delete ctx;
}

extern "C" aexq_status aexq_set_stream(aexq_ctx* ctx, void* hip_stream) {
  if (!ctx) return fail(AEXQ_ERR_INVALID_ARGUMENT, "aexq_set_stream", "ctx is NULL");
  ctx->stream = (hipStream_t)hip_stream;
  return AEXQ_OK;
}

extern "C" aexq_status aexq_synchronize(aexq_ctx* ctx) {
  if (!ctx) return fail(AEXQ_ERR_INVALID_ARGUMENT, "aexq_synchronize", "ctx is NULL");
  HIP_TRY("aexq_synchronize", hipSetDevice(ctx->device));
  HIP_TRY("aexq_synchronize", hipStreamSynchronize(ctx->stream));
  return AEXQ_OK;
}

// ---------------------------------------------------------------------------
// weights
// ---------------------------------------------------------------------------
// A weight's device buffers, codes set to the padding code (0 in device form)
// and scales to zero; the caller fills them.
static aexq_status alloc_weight(aexq_ctx* ctx, const char* op, int bits, int scale_dtype, int n,
                                int k, int block, int nibble_code, aexq_weight** out) {
  aexq_weight* w = new aexq_weight();
  w->device = ctx->device;
  w->bits = bits;
  w->n = n;
  w->k = k;
  w->block = block;
  w->scale_dtype = scale_dtype;
  w->nibble_code = nibble_code;
  const long long count = (long long)n * k;
  const long long words = bits == 8 ? (count + 3) / 4 : (count + 7) / 8;
  w->code_bytes = (words < 1 ? 1 : words) * 4;
  w->scale_count = count / block;
  w->code_stride = round_up(w->code_bytes, 256);
  // at least 16 zeroed bytes after each copy's scales: the MFMA kernels' wide
  // scale loads may run into them
  w->scale_stride = round_up(w->scale_count * scale_bytes(scale_dtype) + 16, 256);
  const int pad_byte = bits == 8 ? 0x80 : 0x88;
  hipError_t e = hipSetDevice(ctx->device);
  if (e == hipSuccess) e = hipMalloc((void**)&w->codes, w->code_stride);
  if (e == hipSuccess) e = hipMalloc(&w->scales, w->scale_stride);
  if (e == hipSuccess) e = hipMemset(w->codes, pad_byte, w->code_stride);
  if (e == hipSuccess) e = hipMemset(w->scales, 0, w->scale_stride);
  if (e != hipSuccess) {
    (void)hipFree(w->codes);
    (void)hipFree(w->scales);
    delete w;
    return hip_fail(e, op, "weight allocation");
  }
  *out = w;
  return AEXQ_OK;
}

// Q4 weights: whether fp16(q * s) stays finite for every code |q| <= 8, from
// the largest scale magnitude (a device reduction over the scales, once at
// upload).  A NaN or infinite scale propagates the same in both GEMM forms.
static aexq_status check_fp16_dequant(aexq_weight* w, const char* op) {
  if (w->bits != 4) return AEXQ_OK;
  unsigned* dev = nullptr;
  unsigned host = 0;
  hipError_t e = hipMalloc((void**)&dev, sizeof(unsigned));
  if (e == hipSuccess) e = hipMemset(dev, 0, sizeof(unsigned));
  if (e == hipSuccess)
    e = scale_absmax_launch(w->scales, w->scale_count, w->scale_dtype == AEXQ_DTYPE_F16, dev,
                            nullptr);
  if (e == hipSuccess) e = hipMemcpy(&host, dev, sizeof(unsigned), hipMemcpyDeviceToHost);
  (void)hipFree(dev);
  if (e != hipSuccess) return hip_fail(e, op, "scale range check");
  float mx;
  memcpy(&mx, &host, sizeof(float));
  w->fp16_dequant_ok = !(mx > 65504.0f / 8.0f);
  return AEXQ_OK;
}

static void free_weight(aexq_weight* w) {
  (void)hipFree(w->codes);
  (void)hipFree(w->scales);
  delete w;
}

static aexq_status upload_weight(aexq_ctx* ctx, const char* op, int bits, const void* packed,
                                 const void* scales, int scale_dtype, int n, int k, int block,
                                 int nibble_code, aexq_weight** out) {
  aexq_weight* w = nullptr;
  aexq_status st = alloc_weight(ctx, op, bits, scale_dtype, n, k, block, nibble_code, &w);
  if (st) return st;
  // Device code layout: Q8 bytes biased by 128 (q + 128), Q4 nibbles offset-8
  // (q + 8).  Both are one XOR of the reference's two's-complement words; the
  // synthetic offset-8 Q4 words are already in device form.
  uint32_t flip = 0u;
  if (bits == 8) flip = 0x80808080u;
  if (bits == 4 && nibble_code == AEXQ_NIBBLE_TWOS) flip = 0x88888888u;
  std::vector<uint32_t> recoded;
  const void* src = packed;
  if (flip) {
    const long long nw = w->code_bytes / 4;
    recoded.resize((size_t)nw);
    const uint32_t* in = (const uint32_t*)packed;
    for (long long i = 0; i < nw; ++i) recoded[(size_t)i] = in[i] ^ flip;
    src = recoded.data();
  }
  hipError_t e = hipMemcpy(w->codes, src, w->code_bytes, hipMemcpyHostToDevice);
  if (e == hipSuccess)
    e = hipMemcpy(w->scales, scales, w->scale_count * scale_bytes(scale_dtype),
                  hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    free_weight(w);
    return hip_fail(e, op, "weight upload");
  }
  st = check_fp16_dequant(w, op);
  if (st) {
    free_weight(w);
    return st;
  }
  *out = w;
  return AEXQ_OK;
}

extern "C" aexq_status aexq_weight_q8(aexq_ctx* ctx, const uint32_t* packed, const void* scales,
                                      int scale_dtype, int n, int k, int block,
                                      aexq_weight** out) {
  const char* op = "aexq_weight_q8";
  if (!ctx || !packed || !scales || !out)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "NULL argument");
  if (n <= 0 || k <= 0)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "n=%d k=%d must be positive", n, k);
  if (scale_dtype != AEXQ_DTYPE_F16 && scale_dtype != AEXQ_DTYPE_F32)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "scale_dtype=%d", scale_dtype);
  if (block == 0) block = k;
  // GL:65-67 / GS:12893-12894: the direct Q8 path needs one scale per output row
  if (block != k)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op,
                "Direct Q8 upload must contain one scale per output channel | block=%d k=%d",
                block, k);
  return upload_weight(ctx, op, 8, packed, scales, scale_dtype, n, k, k, AEXQ_NIBBLE_TWOS, out);
}

extern "C" aexq_status aexq_weight_q4(aexq_ctx* ctx, const uint32_t* packed, const void* scales,
                                      int scale_dtype, int n, int k, int block, int nibble_code,
                                      aexq_weight** out) {
  const char* op = "aexq_weight_q4";
  if (!ctx || !packed || !scales || !out)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "NULL argument");
  if (n <= 0 || k <= 0)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "n=%d k=%d must be positive", n, k);
  if (scale_dtype != AEXQ_DTYPE_F16 && scale_dtype != AEXQ_DTYPE_F32)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "scale_dtype=%d", scale_dtype);
  if (nibble_code != AEXQ_NIBBLE_TWOS && nibble_code != AEXQ_NIBBLE_OFFSET8)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "nibble_code=%d", nibble_code);
  // GS:12979-12980: the group must divide K
  if (block <= 0 || k % block != 0)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op,
                "Direct Q4 group size must divide the Gemm K dimension | block=%d k=%d", block, k);
  return upload_weight(ctx, op, 4, packed, scales, scale_dtype, n, k, block, nibble_code, out);
}

// Unity Mathf.RoundToInt: ties to even; NaN / out of range -> int.MinValue (x64 CLR).
static int round_to_int(float v) {
  const double r = nearbyint((double)v);
  if (isnan(r) || r >= 2147483648.0 || r < -2147483648.0) return INT32_MIN;
  return (int)r;
}
static float unity_max(float a, float b) { return a > b ? a : b; }

// GS:12838-12885 / GS:12912-12964: per output channel symmetric quantization.
// The device copy is always [n][k] (transB); a [k][n] source is transposed
// while packing, which keeps every code and scale identical.
static aexq_status weight_from_f32(aexq_ctx* ctx, const char* op, int bits, const float* data,
                                   int n, int k, int trans_b, aexq_weight** out) {
  if (!ctx || !data || !out) return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "NULL argument");
  if (n <= 0 || k <= 0)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "n=%d k=%d must be positive", n, k);
  const long long count = (long long)n * k;
  const int qmax = bits == 8 ? 127 : 7;
  std::vector<uint32_t> packed(bits == 8 ? (count + 3) / 4 : (count + 7) / 8, 0u);
  std::vector<float> scales(n);
  for (int oc = 0; oc < n; ++oc) {
    float max_abs = 0.0f;
    for (int vi = 0; vi < k; ++vi) {
      const long long src = trans_b ? (long long)oc * k + vi : (long long)vi * n + oc;
      max_abs = unity_max(max_abs, fabsf(data[src]));
    }
    const float scale = max_abs > 0.0f ? max_abs / (float)qmax : 1.0f;
    scales[oc] = scale;
    for (int vi = 0; vi < k; ++vi) {
      const long long src = trans_b ? (long long)oc * k + vi : (long long)vi * n + oc;
      int q = round_to_int(data[src] / scale);
      q = q < -qmax ? -qmax : (q > qmax ? qmax : q);
      const long long dst = (long long)oc * k + vi;
      if (bits == 8)
        packed[dst >> 2] |= (uint32_t)(uint8_t)(int8_t)q << ((dst & 3) * 8);
      else
        packed[dst >> 3] |= ((uint32_t)q & 0xfu) << ((dst & 7) * 4);
    }
  }
  return upload_weight(ctx, op, bits, packed.data(), scales.data(), AEXQ_DTYPE_F32, n, k, k,
                       AEXQ_NIBBLE_TWOS, out);
}

extern "C" aexq_status aexq_weight_q8_from_f32(aexq_ctx* ctx, const float* data, int n, int k,
                                               int trans_b, aexq_weight** out) {
  return weight_from_f32(ctx, "aexq_weight_q8_from_f32", 8, data, n, k, trans_b, out);
}

extern "C" aexq_status aexq_weight_q4_from_f32(aexq_ctx* ctx, const float* data, int n, int k,
                                               int trans_b, aexq_weight** out) {
  return weight_from_f32(ctx, "aexq_weight_q4_from_f32", 4, data, n, k, trans_b, out);
}

// ---------------------------------------------------------------------------
// AQSGET8 archives (Q8A = NcnnQ8Archive.cs): the archive header, and one Gemm
// weight record straight into the device layout.
// ---------------------------------------------------------------------------
static constexpr uint64_t kArchiveMagic = 0x0038544547535141ull;  // Q8A:26 "AQSGET8"
static constexpr uint32_t kArchiveVersion = 1u;                    // Q8A:27
static constexpr uint32_t kRecordMagic = 0x31523851u;              // Q8A:28 "Q8R1"
static constexpr int kRecordQ8 = 1, kRecordRaw = 2, kRecordQ4 = 3;  // Q8A:31-33
static constexpr size_t kRecordHeaderBytes = 24;                   // Q8A:30, 236-245

static uint32_t get_u32(const uint8_t* p) {
  uint32_t v;
  memcpy(&v, p, 4);
  return v;
}

extern "C" aexq_status aexq_archive_header(const void* buf, size_t len, int* quant_bits,
                                           int* default_block, int* record_count) {
  const char* op = "aexq_archive_header";
  if (!buf) return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "buf is NULL");
  const uint8_t* b = (const uint8_t*)buf;
  if (len < 32) return fail(AEXQ_ERR_FORMAT, op, "archive header needs 32 bytes, got %zu", len);
  uint64_t magic;
  memcpy(&magic, b, 8);
  // Q8A:280-290
  if (magic != kArchiveMagic) return fail(AEXQ_ERR_FORMAT, op, "Invalid AIImage Q8 archive magic.");
  const uint32_t version = get_u32(b + 8);
  if (version != kArchiveVersion)
    return fail(AEXQ_ERR_FORMAT, op, "Unsupported AIImage Q8 archive version: %u", version);
  const int bits = (int)get_u32(b + 12);
  const int block = (int)get_u32(b + 16);
  const int records = (int)get_u32(b + 20);
  if (block <= 0 || records < 0 || (bits != 0 && bits != 4 && bits != 8))
    return fail(AEXQ_ERR_FORMAT, op, "Invalid AIImage quantized archive header.");
  if (quant_bits) *quant_bits = bits == 0 ? 8 : bits;  // Q8A:293
  if (default_block) *default_block = block;
  if (record_count) *record_count = records;
  return AEXQ_OK;
}

struct RecordHeader {
  int kind, count, block, payload;
};

// Q8A:447-463 ReadHeader, plus the bounds of the caller's buffer.
static aexq_status read_record_header(const char* op, const uint8_t* rec, size_t len,
                                      long long expected, RecordHeader* h) {
  if (len < kRecordHeaderBytes)
    return fail(AEXQ_ERR_FORMAT, op, "record header needs %zu bytes, got %zu",
                kRecordHeaderBytes, len);
  if (get_u32(rec) != kRecordMagic) return fail(AEXQ_ERR_FORMAT, op, "Invalid Q8 record magic.");
  h->kind = (int)get_u32(rec + 4);
  h->count = (int)get_u32(rec + 8);
  h->block = (int)get_u32(rec + 12);
  h->payload = (int)get_u32(rec + 16);
  if ((long long)h->count != expected)
    return fail(AEXQ_ERR_FORMAT, op, "Q8 record element count mismatch. expected=%lld actual=%d",
                expected, h->count);
  if (h->block <= 0 || h->payload < 0) return fail(AEXQ_ERR_FORMAT, op, "Invalid Q8 record header.");
  if (len - kRecordHeaderBytes < (size_t)h->payload)
    return fail(AEXQ_ERR_FORMAT, op, "record payload of %d bytes, %zu available", h->payload,
                len - kRecordHeaderBytes);
  return AEXQ_OK;
}

// Bytes a Q8 / Q4 record of `count` elements in blocks of `block` consumes
// (Q8A:249-255); the reader requires the header's payload to match (Q8A:465-469).
static long long quant_payload_bytes(int kind, long long count, int block) {
  const long long full = count / block, tail = count - full * block;
  const long long per = kind == kRecordQ8 ? block : (block + 1) / 2;
  long long bytes = full * (4 + per);
  if (tail) bytes += 4 + (kind == kRecordQ8 ? tail : (tail + 1) / 2);
  return bytes;
}

// Q8A:295-339 ReadArray: the record as float32 (raw copied; Q8 (sbyte)b * scale;
// Q4 (raw >= 8 ? raw - 16 : raw) * scale).
static aexq_status record_as_f32(const char* op, const RecordHeader& h, const uint8_t* payload,
                                 std::vector<float>& out) {
  const long long count = h.count;
  out.assign((size_t)count, 0.0f);
  if (h.kind == kRecordRaw) {
    if ((long long)h.payload != count * 4)
      return fail(AEXQ_ERR_FORMAT, op, "Q8 raw float record size mismatch.");
    memcpy(out.data(), payload, (size_t)count * 4);
    return AEXQ_OK;
  }
  if (h.kind != kRecordQ8 && h.kind != kRecordQ4)
    return fail(AEXQ_ERR_FORMAT, op, "Expected a quantized array record.");
  const long long need = quant_payload_bytes(h.kind, count, h.block);
  if (need != h.payload)
    return fail(AEXQ_ERR_FORMAT, op, "Q8 payload size mismatch. expected=%d actual=%lld",
                h.payload, need);
  long long used = 0;
  for (long long off = 0; off < count; off += h.block) {
    const long long len = h.block < count - off ? h.block : count - off;
    float scale;
    memcpy(&scale, payload + used, 4);
    used += 4;
    if (h.kind == kRecordQ8) {
      for (long long i = 0; i < len; ++i) out[off + i] = (float)(int8_t)payload[used + i] * scale;
      used += len;
    } else {
      for (long long i = 0; i < len; ++i) {
        const int raw = (payload[used + (i >> 1)] >> ((i & 1) * 4)) & 0xf;
        out[off + i] = (float)(raw >= 8 ? raw - 16 : raw) * scale;
      }
      used += (len + 1) / 2;
    }
  }
  return AEXQ_OK;
}

extern "C" aexq_status aexq_weight_from_record(aexq_ctx* ctx, int bits, const void* record,
                                               size_t record_len, int n, int k,
                                               aexq_weight** out, size_t* consumed) {
  const char* op = "aexq_weight_from_record";
  if (!ctx || !record || !out) return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "NULL argument");
  if (bits != 4 && bits != 8) return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "bits=%d (4 or 8)", bits);
  if (n <= 0 || k <= 0)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "n=%d k=%d must be positive", n, k);
  const long long count = (long long)n * k;
  if (count > 0x7fffffffLL)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "n*k=%lld exceeds a record's count", count);
  const uint8_t* rec = (const uint8_t*)record;
  RecordHeader h;
  aexq_status st = read_record_header(op, rec, record_len, count, &h);
  if (st) return st;
  const uint8_t* payload = rec + kRecordHeaderBytes;
  if (consumed) *consumed = kRecordHeaderBytes + (size_t)h.payload;
  const bool direct = (bits == 4 && h.kind == kRecordQ4) || (bits == 8 && h.kind == kRecordQ8);
  if (!direct) {
    // GL:60-68: a record of another kind is read as float32 and quantized per
    // output row at upload (GL:113-141 -> GS:12838-12885, 12912-12964)
    std::vector<float> values;
    st = record_as_f32(op, h, payload, values);
    if (st) return st;
    return weight_from_f32(ctx, op, bits, values.data(), n, k, 1, out);
  }
  // Q8A:345-346 / GL:67: the direct Q8 path reads with expectedBlockSize = K
  if (bits == 8 && h.block != k)
    return fail(AEXQ_ERR_FORMAT, op, "Q8 block size mismatch. expected=%d actual=%d", k, h.block);
  // GS:12979-12980
  if (bits == 4 && k % h.block != 0)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op,
                "Direct Q4 group size must divide the Gemm K dimension. | block=%d k=%d", h.block,
                k);
  const long long need = quant_payload_bytes(h.kind, count, h.block);
  if (need != h.payload)
    return fail(AEXQ_ERR_FORMAT, op, "Q8 payload size mismatch. expected=%d actual=%lld",
                h.payload, need);
  aexq_weight* w = nullptr;
  st = alloc_weight(ctx, op, bits, AEXQ_DTYPE_F32, n, k, h.block, AEXQ_NIBBLE_TWOS, &w);
  if (st) return st;
  // the payload goes to the device as it is and is repacked there; the
  // allocation's fills and the repack are ordered on the null stream
  void* staging = nullptr;
  hipError_t e = hipMalloc(&staging, (size_t)h.payload > 0 ? (size_t)h.payload : 1);
  if (e == hipSuccess && h.payload > 0)
    e = hipMemcpy(staging, payload, (size_t)h.payload, hipMemcpyHostToDevice);
  if (e == hipSuccess)
    e = record_repack_launch(staging, count, h.block, bits, w->codes, (float*)w->scales, nullptr);
  if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
  (void)hipFree(staging);
  if (e != hipSuccess) {
    free_weight(w);
    return hip_fail(e, op, "record repack");
  }
  st = check_fp16_dequant(w, op);
  if (st) {
    free_weight(w);
    return st;
  }
  *out = w;
  return AEXQ_OK;
}

extern "C" aexq_status aexq_weight_replicate(aexq_ctx* ctx, const aexq_weight* src, int batch,
                                             aexq_weight** out) {
  const char* op = "aexq_weight_replicate";
  if (!ctx || !src || !out) return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "NULL argument");
  if (src->device != ctx->device)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "weight on device %d, context on device %d",
                src->device, ctx->device);
  if (batch <= 0) return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "batch=%d", batch);
  aexq_weight* w = new aexq_weight(*src);
  w->device = ctx->device;
  w->batch = batch;
  w->owns = true;
  w->codes = nullptr;
  w->scales = nullptr;
  hipError_t e = hipSetDevice(ctx->device);
  if (e == hipSuccess) e = hipMalloc((void**)&w->codes, w->code_stride * batch);
  if (e == hipSuccess) e = hipMalloc(&w->scales, w->scale_stride * batch);
  for (int b = 0; b < batch && e == hipSuccess; ++b) {
    e = hipMemcpy((char*)w->codes + b * w->code_stride, src->codes, src->code_stride,
                  hipMemcpyDeviceToDevice);
    if (e == hipSuccess)
      e = hipMemcpy((char*)w->scales + b * w->scale_stride, src->scales, src->scale_stride,
                    hipMemcpyDeviceToDevice);
  }
  if (e != hipSuccess) {
    (void)hipFree(w->codes);
    (void)hipFree(w->scales);
    delete w;
    return hip_fail(e, op, "replicate");
  }
  *out = w;
  return AEXQ_OK;
}

extern "C" aexq_status aexq_weight_alias(aexq_ctx* ctx, const aexq_weight* shared,
                                         aexq_weight** out) {
  if (!ctx || !shared || !out)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, "aexq_weight_alias", "NULL argument");
  if (shared->device != ctx->device)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, "aexq_weight_alias",
                "weight on device %d, context on device %d", shared->device, ctx->device);
  aexq_weight* w = new aexq_weight(*shared);
  w->owns = false;
  *out = w;
  return AEXQ_OK;
}

extern "C" void aexq_weight_release(aexq_weight* w) {
  if (!w) return;
  if (w->owns) {
    (void)hipSetDevice(w->device);
    (void)hipFree(w->codes);
    (void)hipFree(w->scales);
  }
  delete w;
}

extern "C" aexq_status aexq_weight_get_info(const aexq_weight* w, aexq_weight_info* out) {
  if (!w || !out) return fail(AEXQ_ERR_INVALID_ARGUMENT, "aexq_weight_get_info", "NULL argument");
  out->bits = w->bits;
  out->n = w->n;
  out->k = w->k;
  out->block = w->block;
  out->scale_dtype = w->scale_dtype;
  out->nibble_code = w->nibble_code;
  out->batch = w->batch;
  out->code_bytes = w->code_bytes;
  out->scale_bytes = w->scale_count * scale_bytes(w->scale_dtype);
  return AEXQ_OK;
}

// ---------------------------------------------------------------------------
// tensors
// ---------------------------------------------------------------------------
struct TensorView {
  int rows = 0;          // logical M
  int width = 0;         // logical W
  long long rstride = 0; // elements between rows
  int padded = 0;        // row elements the layout stores (zero-filled tail)
  int batch = 1;
  long long bstride = 0;
  int dtype = AEXQ_DTYPE_F16;
  void* data = nullptr;
  int head_dim = 0;      // attention head-packed layout: head dim and head count
  int heads = 0;
};

static bool same_shape(const aexq_shape& a, int dims, int w, int h, int d, int c) {
  return a.dims == dims && a.w == w && a.h == h && a.d == d && a.c == c;
}

// Storage rules of GS:10818-10857 for the three supported layouts.
static aexq_status view_tensor(const aexq_tensor* t, const char* op, const char* name,
                               TensorView* v) {
  if (!t) return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "%s is NULL", name);
  if (!t->data) return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "%s.data is NULL", name);
  if (t->dtype != AEXQ_DTYPE_F16 && t->dtype != AEXQ_DTYPE_F32)
    return fail(AEXQ_ERR_UNSUPPORTED, op, "%s dtype=%d | rejectedFallback=dtype", name, t->dtype);
  const aexq_shape& L = t->logical;
  // an empty matrix (no columns, or no rows of a 2-D shape) is refused, never
  // launched as one row
  if (L.dims < 1 || L.w <= 0 || (L.dims >= 2 && L.h <= 0))
    return fail(AEXQ_ERR_SHAPE, op, "%s logical {%d,%d,%d,%d,%d} is empty", name, L.dims, L.w,
                L.h, L.d, L.c);
  const int W = L.w;
  const int H = L.dims >= 2 ? L.h : 1;
  v->rows = H;
  v->width = W;
  v->dtype = t->dtype;
  v->data = t->data;
  v->batch = t->batch > 0 ? t->batch : 1;
  v->bstride = t->batch_stride;
  if (L.dims > 2 && (L.d > 1 || L.c > 1))
    return fail(AEXQ_ERR_SHAPE, op, "%s logical dims=%d d=%d c=%d is not a 2-D matrix", name,
                L.dims, L.d, L.c);
  const int packs = (W + 3) / 4;
  switch (t->layout) {
    case AEXQ_LAYOUT_LINEAR:
      if (!(same_shape(t->storage, 2, W, H, 1, 1) || same_shape(t->storage, L.dims, L.w, L.h, L.d, L.c)))
        return fail(AEXQ_ERR_SHAPE, op, "%s LinearMat storage {%d,%d,%d,%d,%d} != logical [%d][%d]",
                    name, t->storage.dims, t->storage.w, t->storage.h, t->storage.d,
                    t->storage.c, H, W);
      v->rstride = W;
      v->padded = W;
      break;
    case AEXQ_LAYOUT_PACK4_LINEAR:
      // ResolvePack4LinearMatStorageShape: {3, ceil(w/4), h, 1, 4}
      if (!same_shape(t->storage, 3, packs, H, 1, 4))
        return fail(AEXQ_ERR_SHAPE, op,
                    "%s Pack4 storage {%d,%d,%d,%d,%d} != {3,%d,%d,1,4}", name, t->storage.dims,
                    t->storage.w, t->storage.h, t->storage.d, t->storage.c, packs, H);
      v->rstride = (long long)packs * 4;
      v->padded = packs * 4;
      break;
    case AEXQ_LAYOUT_PACK4_TILED: {
      // ResolvePack4TiledLinearMatStorageShape: {3, tileWidth, h*tileRows, 1, 4}
      const int tw = t->storage.w;
      if (t->storage.dims != 3 || t->storage.c != 4 || t->storage.d != 1 || tw <= 0 ||
          t->storage.h % H != 0)
        return fail(AEXQ_ERR_SHAPE, op, "%s tiled storage {%d,%d,%d,%d,%d} is not Pack4 tiled",
                    name, t->storage.dims, t->storage.w, t->storage.h, t->storage.d,
                    t->storage.c);
      const int tile_rows = t->storage.h / H;
      if ((long long)tw * tile_rows < packs || tile_rows != (packs + tw - 1) / tw)
        return fail(AEXQ_ERR_SHAPE, op, "%s tiled storage %dx%d cannot hold %d packs", name, tw,
                    tile_rows, packs);
      v->rstride = (long long)tw * tile_rows * 4;
      v->padded = packs * 4;
      break;
    }
    case AEXQ_LAYOUT_HEAD_PACKED: {
      // BufferShape {3, head_dim, rows, 1, heads} (GL:1003-1043): ceil(heads/4)
      // slices of rows x head_dim texels, lane head % 4 (MM:1192-1389)
      const aexq_shape& S = t->storage;
      if (S.dims != 3 || S.d != 1 || S.w <= 0 || S.c <= 0 || S.h != H ||
          (long long)S.w * S.c != W)
        return fail(AEXQ_ERR_SHAPE, op,
                    "%s head-packed storage {%d,%d,%d,%d,%d} != {3,head_dim,%d,1,heads} with "
                    "head_dim*heads=%d",
                    name, S.dims, S.w, S.h, S.d, S.c, H, W);
      v->head_dim = S.w;
      v->heads = S.c;
      v->rstride = 0;  // not row-major
      v->padded = (S.c + 3) / 4 * 4 * S.w;
      break;
    }
    default:
      return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "%s layout=%d", name, t->layout);
  }
  return AEXQ_OK;
}

// ---------------------------------------------------------------------------
// strict plan
// ---------------------------------------------------------------------------
enum PlanKind : int { kPlanGeneric = 0, kPlanStream = 1, kPlanMfma = 2, kPlanGemm = 3 };

struct Plan {
  int kind = kPlanGeneric;
  bool fast = false;                 // streaming matvec kernel
  const QmvEntry* entry = nullptr;   // streaming kernel
  const QmmEntry* mentry = nullptr;  // MFMA kernel
  const QgemmEntry* gentry = nullptr;  // tiled GEMM (M > 32)
  int fmt = kQ8;
  int rows_per_tile = 0;
  QmvParams p{};
  int grid = 0;
  // MFMA path: RMSNorm-in runs as a row pre-pass into the context's
  // activation scratch; rows go in blocks of `mblock` per launch
  bool rms_prepass = false;
  int mblock = 0;
  int x_f32 = 0;
  int x_batch = 1;
  long long x_rstride_in = 0;
  long long x_bstride_in = 0;
  int ysz = 2;
  // head-packed x: gathered into dense rows (the context's gather scratch) first
  bool x_gather = false;
  const void* xg_src = nullptr;
  int xg_heads = 0, xg_hd = 0, xg_rows = 0, xg_batch = 1, xg_f32 = 0;
  long long xg_bstride = 0;
  // split K (MFMA kernels): sk_chunks chunks of sk_cs K steps per tile, partials
  // summed by the fix-up launch; sk_nw = 2 for a SwiGLU pair
  int sk_chunks = 1, sk_cs = 0, sk_nw = 1;
};

// Split K for an MFMA launch of `units` independent tiles of `steps` K steps
// on at most `slots` resident workgroups: the chunk count with the least
// estimated time -- the rounds of whole workgroups times the K steps each
// runs (step_us per step, measured per kernel family: these launches wait on
// load latency, not on bandwidth), plus, once split, the fix-up launch and the
// fp32 partials written and read back (plane_bytes per chunk).  A layer's
// linear at M = 16..512 has few tiles (8 for a 1024-row output), so without
// the split a handful of workgroups would walk all of K on a 256-CU part.
// AEXQ_SPLITK=n forces n chunks (1: no split).
static void pick_split(long long units, int steps, long long slots, double step_us,
                       double wg_us, int max_chunks, double plane_bytes, int* chunks, int* cs) {
  constexpr double kFixupUs = 5.0;         // the fix-up launch and its round trips
  constexpr double kPartBytesPerUs = 5e6;  // partial planes written and read back
  constexpr double kMaxPartBytes = 256.0 * 1024 * 1024;
  *chunks = 1;
  *cs = steps;
  if (steps < 2 || units < 1 || slots < 1) return;
  const char* env = getenv("AEXQ_SPLITK");
  if (env && atoi(env) >= 1) {
    int want = atoi(env) < steps ? atoi(env) : steps;
    // within the same partial-plane budget as the model's choice
    const long long fit = plane_bytes > 0 ? (long long)(kMaxPartBytes / plane_bytes) : steps;
    if (want > fit) want = fit > 1 ? (int)fit : 1;
    *cs = (steps + want - 1) / want;
    *chunks = (steps + *cs - 1) / *cs;
    if (*chunks < 2) *cs = steps;
    return;
  }
  double best = 0.0;
  for (int c = 1; c <= steps; ++c) {
    const int w = (steps + c - 1) / c;  // steps per chunk
    const int n = (steps + w - 1) / w;  // chunks that takes
    if (n != c) continue;               // same chunking as a smaller count
    if (n > 1 && (n * plane_bytes > kMaxPartBytes || n > max_chunks)) break;
    const long long work = units * n;
    const long long rounds = (work + slots - 1) / slots;
    double t = (double)rounds * (w * step_us + wg_us);
    if (n > 1) t += kFixupUs + n * plane_bytes * 2.0 / kPartBytesPerUs;
    if (c == 1 || t < best) {
      best = t;
      *chunks = n;
      *cs = w;
    }
  }
  if (*chunks < 2) {
    *chunks = 1;
    *cs = steps;
  }
}

// Partial-plane layout of one split launch (per-matrix offsets, plane size in
// floats, 256-byte aligned planes).
static long long splitk_layout(QmvParams& q, int nw) {
  long long off = 0;
  for (int i = 0; i < q.nmat; ++i) {
    q.mat[i].sk_off = off;
    off += (long long)q.batch * q.m * nw * q.mat[i].n_store;
  }
  q.sk_plane = (off + 63) & ~63LL;
  return q.sk_plane;
}

// Shape of the streaming kernel for `chunks` 16-byte code chunks per row:
// the smallest lanes-per-row x chunks-per-lane capacity that covers the row,
// then the fewest lanes per row whose activation registers (chunks per lane x
// 8 or 16 dwords per row of M) stay within 32 dwords per activation row.
// AEXQ_QMV_SHAPE=lpr:cpl overrides the choice (tuning).
static bool pick_shape(int fmt, int chunks, int mmax, int* lpr, int* cpl) {
  const int xw = fmt == kQ8 ? 8 : 16;
  const char* env = getenv("AEXQ_QMV_SHAPE");
  if (env) {
    int a = 0, b = 0;
    if (sscanf(env, "%d:%d", &a, &b) == 2 && a * b >= chunks) {
      *lpr = a;
      *cpl = b;
      return true;
    }
  }
  const int lprs[3] = {16, 32, 64};
  const int cpls[3] = {1, 2, 4};
  int best_cap = 0, best_fit = 0, best_l = 0, best_c = 0;
  for (int li = 0; li < 3; ++li)
    for (int ci = 0; ci < 3; ++ci) {
      const int l = lprs[li], c = cpls[ci];
      // M > 1 shapes: one chunk per lane (Q8 also 64 x 2)
      if (mmax > 1 && c > 1 && !(fmt == kQ8 && l == 64 && c == 2)) continue;
      const int cap = l * c;
      if (cap < chunks) continue;
      const int fit = c * xw <= 32 ? 0 : 1;
      // lexicographic: capacity, register fit, lanes per row
      const bool better = !best_l || cap < best_cap || (cap == best_cap && fit < best_fit) ||
                          (cap == best_cap && fit == best_fit && l < best_l);
      if (better) {
        best_cap = cap;
        best_fit = fit;
        best_l = l;
        best_c = c;
      }
    }
  if (!best_l) return false;
  *lpr = best_l;
  *cpl = best_c;
  return true;
}

static const char* kLinearOp = "aexq_linear";

static aexq_status make_plan(aexq_ctx* ctx, int count, const aexq_weight* const* ws,
                             const aexq_tensor* x, const aexq_tensor* const* ys,
                             const aexq_linear_args* args, bool argmax, Plan* plan) {
  const char* op = argmax ? "aexq_lmhead_argmax" : kLinearOp;
  if (!ctx) return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "ctx is NULL");
  if (count <= 0 || count > kMaxGroup)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "group count=%d (1..%d)", count, kMaxGroup);
  aexq_linear_args def{};
  def.alpha = 1.0f;
  def.beta = 1.0f;
  def.broadcast_c = -1;
  def.rms_eps = 0.001f;
  const aexq_linear_args& a = args ? *args : def;
  const unsigned known = AEXQ_EPI_RMSNORM_IN | AEXQ_EPI_SWIGLU_OUT | AEXQ_EPI_RESIDUAL_ADD |
                         AEXQ_EPI_EXACT_DEQUANT | (argmax ? AEXQ_EPI_ARGMAX_F16 : 0u);
  if (a.flags & ~known)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "flags=0x%x%s", a.flags,
                (a.flags & AEXQ_EPI_ARGMAX_F16) && !argmax ? " (ARGMAX_F16 is for the LM head)" : "");
  const aexq_weight* w0 = ws[0];
  if (!w0) return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "weight is NULL");
  for (int i = 0; i < count; ++i)
    if (ws[i] && ws[i]->device != ctx->device)
      return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "weight %d is on device %d, context on device %d",
                  i, ws[i]->device, ctx->device);
  if (args && args->up && args->up->device != ctx->device)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "up weight is on device %d, context on device %d",
                args->up->device, ctx->device);
  for (int i = 1; i < count; ++i) {
    if (!ws[i]) return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "weight %d is NULL", i);
    if (ws[i]->bits != w0->bits || ws[i]->k != w0->k || ws[i]->batch != w0->batch ||
        ws[i]->block != w0->block || ws[i]->scale_dtype != w0->scale_dtype ||
        ws[i]->nibble_code != w0->nibble_code)
      return fail(AEXQ_ERR_UNSUPPORTED, op,
                  "group member %d differs in bits/k/batch/block/scales | rejectedFallback=group", i);
  }
  const bool swiglu = (a.flags & AEXQ_EPI_SWIGLU_OUT) != 0;
  if (swiglu) {
    if (count != 1) return fail(AEXQ_ERR_UNSUPPORTED, op, "SwiGLU-out takes one gate/up pair");
    const aexq_weight* up = a.up;
    if (!up) return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "SwiGLU-out without the up weight");
    if (up->bits != w0->bits || up->n != w0->n || up->k != w0->k || up->batch != w0->batch ||
        up->block != w0->block || up->scale_dtype != w0->scale_dtype ||
        up->nibble_code != w0->nibble_code || up->code_stride != w0->code_stride ||
        up->scale_stride != w0->scale_stride)
      return fail(AEXQ_ERR_SHAPE, op, "SwiGLU gate/up weights differ in shape or format");
    if (a.c) return fail(AEXQ_ERR_UNSUPPORTED, op, "SwiGLU-out with a C (bias) term");
  }
  if (argmax && (swiglu || (a.flags & AEXQ_EPI_RESIDUAL_ADD)))
    return fail(AEXQ_ERR_UNSUPPORTED, op, "LM head takes no SwiGLU/residual epilogue");
  // one argmax per activation row: the partials carry no batch index
  if (argmax && w0->batch != 1)
    return fail(AEXQ_ERR_UNSUPPORTED, op, "LM head over a batched weight (batch=%d)", w0->batch);
  if (argmax && a.c)
    return fail(AEXQ_ERR_UNSUPPORTED, op, "LM head with a C (bias) term | rejectedFallback=bias");

  TensorView xv;
  aexq_status st = view_tensor(x, op, "x", &xv);
  if (st) return st;
  if (xv.head_dim) {
    if (argmax)
      return fail(AEXQ_ERR_UNSUPPORTED, op, "LM head x in the head-packed layout");
    // gathered at launch into dense rows [batch][M][W]; plan over that view
    plan->x_gather = true;
    plan->xg_src = xv.data;
    plan->xg_heads = xv.heads;
    plan->xg_hd = xv.head_dim;
    plan->xg_rows = xv.rows;
    plan->xg_batch = xv.batch;
    plan->xg_bstride = xv.bstride;
    plan->xg_f32 = xv.dtype == AEXQ_DTYPE_F32;
    xv.rstride = xv.width;
    xv.padded = xv.width;
    xv.bstride = (long long)xv.rows * xv.width;
    xv.data = ctx->gather_scratch ? ctx->gather_scratch : (void*)(uintptr_t)256;  // bound at launch
    xv.head_dim = xv.heads = 0;
  }
  const int K = w0->k;
  if (xv.width != K)
    return fail(AEXQ_ERR_SHAPE, op, "x width=%d != weight K=%d | layer=Gemm", xv.width, K);
  const int M = xv.rows;
  if (xv.batch != 1 && xv.batch != w0->batch)
    return fail(AEXQ_ERR_SHAPE, op, "x batch=%d vs weight batch=%d", xv.batch, w0->batch);

  // output views
  TensorView yv[kMaxGroup];
  for (int i = 0; i < count; ++i) {
    if (!ys[i]) {
      if (!argmax) return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "y %d is NULL", i);
      yv[i] = TensorView{};
      yv[i].rows = M;
      yv[i].width = ws[i]->n;
      yv[i].rstride = ws[i]->n;
      yv[i].padded = ws[i]->n;
      yv[i].dtype = AEXQ_DTYPE_F32;
      continue;
    }
    st = view_tensor(ys[i], op, "y", &yv[i]);
    if (st) return st;
    if (yv[i].width != ws[i]->n || yv[i].rows != M)
      return fail(AEXQ_ERR_SHAPE, op, "y %d is [%d][%d], expected [%d][%d]", i, yv[i].rows,
                  yv[i].width, M, ws[i]->n);
    if (yv[i].batch != w0->batch)
      return fail(AEXQ_ERR_SHAPE, op, "y batch=%d vs weight batch=%d", yv[i].batch, w0->batch);
    if (yv[i].dtype != yv[0].dtype)
      return fail(AEXQ_ERR_UNSUPPORTED, op, "group outputs differ in dtype");
    if (ys[i]->layout != ys[0]->layout)
      return fail(AEXQ_ERR_UNSUPPORTED, op, "group outputs differ in layout");
  }
  if (argmax && yv[0].dtype != AEXQ_DTYPE_F32 && yv[0].dtype != AEXQ_DTYPE_F16)
    return fail(AEXQ_ERR_UNSUPPORTED, op, "LM-head logits must be fp32 or fp16");
  if (yv[0].head_dim && (argmax || (a.flags & AEXQ_EPI_RESIDUAL_ADD)))
    return fail(AEXQ_ERR_UNSUPPORTED, op,
                "head-packed y with %s | rejectedFallback=attention-head-packed Gemm",
                argmax ? "the LM head" : "a residual add");
  TensorView rv;
  if (a.flags & AEXQ_EPI_RESIDUAL_ADD) {
    st = view_tensor(a.residual, op, "residual", &rv);
    if (st) return st;
    if (rv.rows != M || rv.width != yv[0].width || rv.dtype != yv[0].dtype ||
        rv.rstride != yv[0].rstride || count != 1)
      return fail(AEXQ_ERR_SHAPE, op, "residual must match y in shape, layout and dtype");
  }
  if (a.c) {
    if (a.broadcast_c != -1 && a.broadcast_c != 0 && a.broadcast_c != 1 && a.broadcast_c != 2 &&
        a.broadcast_c != 3 && a.broadcast_c != 4)
      return fail(AEXQ_ERR_UNSUPPORTED, op, "Gemm broadcast_type_C unsupported: %d",
                  a.broadcast_c);
    if (count != 1 && (a.broadcast_c == 3 || a.broadcast_c == 4))
      return fail(AEXQ_ERR_UNSUPPORTED, op, "per-column C in a grouped launch");
  }
  if (a.flags & AEXQ_EPI_RMSNORM_IN) {
    if (a.rms_gamma && a.rms_gamma_size <= 0)
      return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "rms_gamma_size=%d", a.rms_gamma_size);
  }

  // ---- kernel selection (no fallback to anything but another GPU kernel)
  const int fmt = w0->bits == 8 ? kQ8 : kQ4;
  const bool chunked = fmt == kQ8 ? (K % 16 == 0) : (K % 32 == 0);
  const int chunks = chunked ? (fmt == kQ8 ? K / 16 : K / 32) : 0;
  const int gmode = fmt == kQ8 ? kGRow : (w0->block == 16 ? kG16 : kG32);
  const bool group_ok = fmt == kQ8 || w0->block == 16 || (w0->block % 32 == 0);
  const bool x_ok = xv.dtype == AEXQ_DTYPE_F16 && xv.rstride % 8 == 0 &&
                    ((uintptr_t)xv.data % 16) == 0 && (xv.batch == 1 || xv.bstride % 8 == 0);
  const bool m_ok = M <= 8;
  // MFMA path (M >= 2): 128-wide K slices, one scale per row or per 16/32 codes,
  // fp16 activation rows (RMSNorm-in makes them in a pre-pass)
  const bool rms_in = (a.flags & AEXQ_EPI_RMSNORM_IN) != 0;
  const bool mfma_ok = M >= 2 && K % 128 == 0 &&
                       (fmt == kQ8 || w0->block == 16 || w0->block == 32) &&
                       (rms_in || (xv.dtype == AEXQ_DTYPE_F16 && xv.rstride % 2 == 0 &&
                                   ((uintptr_t)xv.data % 4) == 0 &&
                                   (xv.batch == 1 || xv.bstride % 2 == 0)));
  // the streaming kernels read gamma[0..K) directly (no index clamp)
  const bool rms_ok = !(a.flags & AEXQ_EPI_RMSNORM_IN) || !a.rms_gamma ||
                      (a.rms_gamma_size >= K && ((uintptr_t)a.rms_gamma % 4) == 0);
  // 32-bit buffer offsets inside one weight copy (and below the kernels' no-chunk offset)
  const bool size_ok = (long long)w0->n * K * w0->bits / 8 < (1LL << 30);
  plan->fmt = fmt;
  plan->fast = false;
  // M > 32: the tiled GEMM (every row of a weight tile per workgroup pass),
  // 64-wide K steps, fp16 activation rows 16-byte aligned; Q4 scale groups of
  // 16 (the reference's shipping Q4) or a multiple of 32
  const bool g16 = fmt == kQ4 && w0->block == 16;
  const bool gemm_shape_ok = K % 64 == 0 && (fmt == kQ8 || w0->block % 32 == 0 || g16) &&
                             (rms_in || x_ok) && size_ok && !argmax &&
                             getenv("AEXQ_QGEMM_OFF") == nullptr;
  // Q4 weight tiles dequantised to fp16 in the tiled GEMM unless the call asks
  // for the exact form or a weight's scales could overflow fp16 there
  bool fd = fmt == kQ4 && !(a.flags & AEXQ_EPI_EXACT_DEQUANT);
  for (int i = 0; i < count && fd; ++i) fd = ws[i]->fp16_dequant_ok;
  if (fd && swiglu) fd = a.up->fp16_dequant_ok;
  auto try_gemm = [&]() {
    const bool sf16 = w0->scale_dtype == AEXQ_DTYPE_F16;
    // the LDS-direct kernel: Q8 and Q4 groups of 16 or 32; larger Q4 groups
    // (multiples of 32) the register-staged one, 64-row tiles
    QgemmConfig gc{fmt, 64, swiglu, sf16, false, false, false};
    if (fmt == kQ8 || w0->block == 16 || w0->block == 32) {
      int bm = M <= 64 ? 64 : 128;
      const char* benv = getenv("AEXQ_QGEMM_BM");  // tuning override: 64 or 128
      if (benv && (atoi(benv) == 64 || atoi(benv) == 128)) bm = atoi(benv);
      // Q4 fp16 tiles at 64-row tiles take 128-wide K steps: a lane's code
      // load is then a whole 16-byte quarter of a 64-byte row step, half the
      // code and scale requests per K of 64-wide steps (the M = 64 launches
      // wait on those requests).  AEXQ_QGEMM_K64 keeps 64-wide steps (tuning).
      const bool k128 = fmt == kQ4 && fd && bm == 64 && K % 128 == 0 &&
                        getenv("AEXQ_QGEMM_K64") == nullptr;
      gc = QgemmConfig{fmt, bm, swiglu, sf16, g16, true, fd, k128};
    }
    plan->gentry = qgemm_find(gc);
    if (plan->gentry) {
      plan->kind = kPlanGemm;
      plan->rms_prepass = rms_in;
    }
  };
  if (M > 32 && gemm_shape_ok) try_gemm();
  if (plan->kind != kPlanGemm && mfma_ok && size_ok) {
    const int mt = M <= 16 ? 1 : 2;
    // 256-wide K steps whose code fetches cover 128 contiguous bytes of 8 rows
    // per instruction, where K and the scale layout allow
    const bool wide = K % 256 == 0 && (fmt == kQ8 || gmode == kG32 || gmode == kG16) &&
                      getenv("AEXQ_QMM_NARROW") == nullptr;
    const int nt = swiglu ? (mt == 1 ? 2 : 1) : (mt == 1 ? 4 : 2);
    QmmConfig mc{fmt, gmode, mt, nt, swiglu, w0->scale_dtype == AEXQ_DTYPE_F16, false, false};
    if (wide) {
      QmmConfig wc = mc;
      wc.wide = true;
      if (fmt == kQ8 && mt == 1) wc.nt = nt > 1 ? nt / 2 : 1;
      if (gmode == kG16) wc.nt = nt > 1 ? nt / 2 : 1;  // twice the scales per block
      if (argmax) {
        // the LM head: argmax partials fused, one 16-row block per wave (two
        // blocks need 208 VGPRs against 150, and ran config 5 at M = 8 in
        // 57-65 us against 45-56 at grids of 2-6 workgroups per CU).  The plain
        // kernel's logits and an argmax launch over them measured no faster
        // (config 5, M = 8: 46-47 us against 45-47): a second launch costs as
        // much as the fused form's epilogue and merge.
        wc.argmax = true;
        wc.nt = 1;
      }
      plan->mentry = qmm_find(wc);
    }
    if (!plan->mentry) plan->mentry = qmm_find(mc);
    if (plan->mentry) {
      plan->kind = kPlanMfma;
      plan->rms_prepass = rms_in;
      plan->mblock = 16 * mt;
    }
  }
  // M = 9..32 where the MFMA block kernel does not apply (K a multiple of 64
  // but not of 128, Q4 scale groups of 64 or more): the tiled GEMM, its rows
  // past M masked, rather than the generic kernel
  if (plan->kind != kPlanMfma && plan->kind != kPlanGemm && M > 8 && gemm_shape_ok) try_gemm();
  if (plan->kind != kPlanMfma && plan->kind != kPlanGemm && chunked && group_ok && x_ok && m_ok && rms_ok && size_ok &&
      chunks > 0) {
    const int mmax = M == 1 ? 1 : 8;
    int lpr = 0, cpl = 0;
    if (pick_shape(fmt, chunks, mmax, &lpr, &cpl)) {
      int u = cpl >= 4 ? 1 : (cpl == 2 ? 2 : 4);
      if (swiglu && u > 1) u /= 2;  // two weights stream per row
      QmvConfig cfg{fmt, lpr, cpl, mmax == 1 ? u : 1, mmax, swiglu, argmax, gmode};
      plan->entry = qmv_find(cfg);
      if (!plan->entry && argmax) {
        cfg.argmax = false;  // logits by the streaming kernel, argmax as a second pass
        plan->entry = qmv_find(cfg);
      }
      plan->fast = plan->entry != nullptr;
      if (plan->fast) plan->kind = kPlanStream;
    }
  }
  if (plan->kind == kPlanGemm) {
    plan->rows_per_tile = qgemm_rows_per_tile(swiglu);
  } else if (plan->kind == kPlanMfma) {
    plan->rows_per_tile = plan->mentry->tn;
  } else if (plan->fast) {
    plan->rows_per_tile = plan->entry->rw;
  } else {
    if (swiglu)
      return fail(AEXQ_ERR_UNSUPPORTED, op,
                  "SwiGLU-out needs fp16 x and K aligned to 16-byte code chunks at M<=8, to 64 "
                  "at larger M | K=%d M=%d "
                  "| rejectedFallback=SwiGLU",
                  K, M);
    plan->rows_per_tile = generic_rows_per_wg();
  }

  // ---- parameters
  QmvParams& p = plan->p;
  p = QmvParams{};
  p.nmat = count;
  p.batch = w0->batch;
  p.k = K;
  p.m = M;
  p.group = w0->block;
  p.groups_per_row = K / w0->block;
  p.chunks = chunks;
  p.x_rstride = xv.rstride;
  p.r_rstride = (a.flags & AEXQ_EPI_RESIDUAL_ADD) ? rv.rstride : 0;
  p.alpha = a.alpha;
  p.beta = a.beta;
  p.c = a.c;
  p.bcast = a.c ? a.broadcast_c : -1;
  p.c_rstride = w0->n;
  p.gamma = (a.flags & AEXQ_EPI_RMSNORM_IN) ? a.rms_gamma : nullptr;
  p.gamma_size = a.rms_gamma_size;
  p.eps = a.rms_eps;
  int flags = 0;
  if (a.flags & AEXQ_EPI_RMSNORM_IN) flags |= kFlagRms;
  if (a.flags & AEXQ_EPI_RESIDUAL_ADD) flags |= kFlagResidual;
  if (yv[0].dtype == AEXQ_DTYPE_F32) flags |= kFlagYf32;
  // MM:1101 (Pack4 linear / LinearMat) vs MM:2301 (tiled)
  const int ylayout = ys[0] ? ys[0]->layout : AEXQ_LAYOUT_LINEAR;
  if (ylayout != AEXQ_LAYOUT_PACK4_TILED) flags |= kFlagAlphaIn;
  if (w0->scale_dtype == AEXQ_DTYPE_F16) flags |= kFlagScaleF16;
  if (xv.dtype == AEXQ_DTYPE_F32) flags |= kFlagXf32;
  // the reference's argmax reads its logits texture: ARGBHalf holds fp16 values
  if (argmax && ((a.flags & AEXQ_EPI_ARGMAX_F16) || yv[0].dtype == AEXQ_DTYPE_F16))
    flags |= kFlagArgF16;
  p.flags = flags;

  int tiles_total = 0;
  for (int i = 0; i < count; ++i) {
    const aexq_weight* w = ws[i];
    QmvMat& mt = p.mat[i];
    mt.w = w->codes;
    mt.s = w->scales;
    mt.w2 = swiglu ? a.up->codes : nullptr;
    mt.s2 = swiglu ? a.up->scales : nullptr;
    mt.x = xv.data;
    mt.y = ys[i] ? yv[i].data : nullptr;
    mt.res = (a.flags & AEXQ_EPI_RESIDUAL_ADD) ? rv.data : nullptr;
    mt.w_bstride = w->code_stride / 4;
    mt.s_bstride = w->scale_stride / scale_bytes(w->scale_dtype);
    mt.x_bstride = xv.batch == 1 ? 0 : xv.bstride;
    mt.y_bstride = ys[i] ? yv[i].bstride : 0;
    mt.r_bstride = (a.flags & AEXQ_EPI_RESIDUAL_ADD) ? rv.bstride : 0;
    mt.y_rstride = yv[i].rstride;
    mt.y_hd = yv[i].head_dim;
    mt.n = w->n;
    mt.n_store = ys[i] ? yv[i].padded : w->n;
    mt.tiles = (mt.n_store + plan->rows_per_tile - 1) / plan->rows_per_tile;
    mt.tile_base = tiles_total;
    const long long add = (long long)mt.tiles * w->batch;
    if (tiles_total + add > 0x7fffffffLL) return fail(AEXQ_ERR_UNSUPPORTED, op, "grid too large");
    tiles_total += (int)add;
  }
  p.total_tiles = tiles_total;
  p.y_rows = M;
  // M = 1 RMSNorm-in over one activation row (not batched; a group shares x):
  // each workgroup stages the normalised row once in LDS (rows up to
  // kQmvStageMaxK; longer ones are normalised by every wave in registers)
  if (plan->kind == kPlanStream && M == 1 && xv.batch == 1 && K <= kQmvStageMaxK &&
      (p.flags & kFlagRms))
    p.flags |= kFlagXShared;
  plan->x_f32 = xv.dtype == AEXQ_DTYPE_F32;
  plan->x_batch = xv.batch;
  plan->x_rstride_in = xv.rstride;
  plan->x_bstride_in = xv.batch == 1 ? 0 : xv.bstride;
  plan->ysz = yv[0].dtype == AEXQ_DTYPE_F32 ? 4 : 2;
  if (plan->kind == kPlanMfma || plan->kind == kPlanGemm) {
    p.flags &= ~kFlagRms;  // normalised by the pre-pass
    if (plan->rms_prepass) {
      // the scratch rows: [x batch][M][K] fp16 (pointer bound at launch)
      p.x_rstride = K;
      for (int i = 0; i < count; ++i) p.mat[i].x_bstride = xv.batch == 1 ? 0 : (long long)M * K;
    }
  }
  const int nw = swiglu ? 2 : 1;
  plan->sk_nw = nw;
  if (plan->kind == kPlanGemm) {
    const int bm = plan->gentry->cfg.bm;
    const int mtiles = (M + bm - 1) / bm;
    plan->mblock = bm;
    const long long slots = (long long)qgemm_blocks_per_cu(plan->gentry) * ctx->cus;
    // per-step and per-workgroup (prologue, epilogue or partial spill) times
    // measured on single-layer launches (graph replays) and s_memrealtime
    // stamps of the LDS-direct kernel
    double step_us, wg_us = 0.0;
    if (plan->gentry->cfg.direct) {
      step_us = fmt == kQ8 ? (bm == 128 ? 0.9 : 0.6)
                           : (g16 ? (bm == 128 ? 2.0 : 1.4) : (bm == 128 ? 1.4 : 1.0));
      wg_us = 3.0;
    } else {
      step_us = 0.9;
    }
    // (at most 8 chunks for the LDS-direct kernel: single layers at M = 64
    // and 512 measured fastest at 4 to 8, slower at 14 to 28)
    const int kstep = plan->gentry->cfg.k128 ? 128 : 64;  // K per step of the kernel
    if (plan->gentry->cfg.k128) step_us *= 2.0;
    pick_split((long long)tiles_total * mtiles, K / kstep, slots, step_us, wg_us,
               plan->gentry->cfg.direct ? 8 : 1 << 30,
               (double)M * nw * tiles_total * plan->rows_per_tile * 4.0,
               &plan->sk_chunks, &plan->sk_cs);
    plan->grid = (int)(((long long)tiles_total + 7) / 8 * 8 * mtiles * plan->sk_chunks);
  } else if (plan->kind == kPlanMfma) {
    int per_cu = qmm_blocks_per_cu(plan->mentry);
    const char* env = getenv("AEXQ_QMM_BLOCKS_PER_CU");
    if (env && atoi(env) > 0) per_cu = atoi(env);
    const long long cap = (long long)per_cu * ctx->cus;
    // both kernels split K where their few tiles would leave the part idle
    // (never for the argmax partials, which need each tile whole); the wide
    // kernel runs a tile per workgroup, the narrow one a tile per wave
    const bool wide = plan->mentry->cfg.wide;
    if (!plan->mentry->cfg.argmax)
      pick_split(tiles_total, K / (wide ? 256 : 128), wide ? cap : cap * kWaves,
                 wide ? (fmt == kQ4 ? 2.2 : 1.15) : 1.0, 0.0, 1 << 30,
                 (double)M * nw * tiles_total * plan->rows_per_tile * 4.0, &plan->sk_chunks,
                 &plan->sk_cs);
    const long long items = (long long)tiles_total * plan->sk_chunks;
    const long long need = wide ? items : (items + kWaves - 1) / kWaves;
    // Q8 on the wide kernel streams best with 6 workgroups per CU queued
    // (config 4, M = 16: 5.35 TB/s at the resident 2, 5.71 at 6); Q4 with the
    // resident count (3.80 at 2, 3.36 at 6), and so does the fused LM head
    // (config 5, M = 8: 45 us at the resident 3, 48 at 2, 56 at 4, 53 at 6)
    long long grid_cap = cap;
    if (wide && fmt == kQ8 && !plan->mentry->cfg.argmax && !env && per_cu < 6)
      grid_cap = 6LL * ctx->cus;
    plan->grid = (int)(need < grid_cap ? need : grid_cap);
    if (plan->grid < 1) plan->grid = 1;
    // RMSNorm-in inside the wide kernel when every item has its own workgroup
    // (the row pre-pass would be a launch of its own, ~4 us, next to a few
    // microseconds of kernel): fp16 rows 16-byte aligned, K within the LDS
    // gamma stage; AEXQ_RMS_PREPASS keeps the pre-pass
    if (wide && plan->rms_prepass && !plan->mentry->cfg.argmax && items <= grid_cap && x_ok &&
        K <= 4096 && K % 8 == 0 && getenv("AEXQ_RMS_PREPASS") == nullptr) {
      QmmConfig rc = plan->mentry->cfg;
      rc.rmsx = true;
      const QmmEntry* re = qmm_find(rc);
      if (re) {
        plan->mentry = re;
        plan->rms_prepass = false;
        p.x_rstride = xv.rstride;
        for (int i = 0; i < count; ++i) p.mat[i].x_bstride = xv.batch == 1 ? 0 : xv.bstride;
      }
    }
  } else if (plan->fast) {
    // persistent grid: every wave resident, each owning a contiguous tile range
    // Workgroups queued beyond the resident count stream best: Q4 16 of 4
    // waves per CU (config 2, against 6, 8, 12, 20, 24 and 32), Q8 12 (config
    // 1, against the resident count, 8 and 16).  Argmax launches take two
    // workgroups per CU, fewer than the resident four (config 5, M = 1: 33.9
    // us against 34.1-34.4 at four, 36.0 at 8 and 46.5 at 16): their waves
    // split the vocabulary by rows, and every workgroup pays its prologue and
    // partial store.
    int per_cu = qmv_blocks_per_cu(plan->entry);
    const bool fused_argmax = plan->entry->cfg.argmax;
    if (fused_argmax) {
      if (per_cu > 2) per_cu = 2;
    } else {
      const int queued = fmt == kQ4 ? 16 : 12;
      if (per_cu < queued) per_cu = queued;
    }
    const char* env = getenv("AEXQ_QMV_BLOCKS_PER_CU");
    if (env && atoi(env) > 0) per_cu = atoi(env);
    const long long need = ((long long)tiles_total + kWaves - 1) / kWaves;
    long long cap = (long long)per_cu * ctx->cus;
    if (fused_argmax) {
      // every workgroup's logits fit its LDS buffer: at most kArgLogitsMax
      // (rows x M) per workgroup, the rows (Pack4 padding included) split
      // evenly over the workgroups
      const long long rows_max = kArgLogitsMax / plan->entry->cfg.mmax;
      const long long g = ((long long)p.mat[0].n_store + rows_max - 1) / rows_max;
      if (g > cap) cap = g;
    }
    plan->grid = (int)(need < cap ? need : cap);
    if (plan->grid < 1) plan->grid = 1;
  } else {
    plan->grid = tiles_total;
  }
  return AEXQ_OK;
}

// MFMA path: optional RMSNorm pre-pass, then one launch per block of rows.
static aexq_status launch_mfma(aexq_ctx* ctx, Plan& plan, const char* op) {
  QmvParams p = plan.p;
  const int M = p.m, K = p.k;
  if (plan.rms_prepass) {
    const long long need = (long long)plan.x_batch * M * K * 2;
    aexq_status st = grow_scratch(ctx, &ctx->act_scratch, &ctx->act_cap, need, op,
                                  "RMSNorm-in rows");
    if (st) return st;
    hipError_t e = rmsnorm_rows_launch(p.mat[0].x, plan.x_f32, plan.x_rstride_in,
                                       plan.x_bstride_in, plan.x_batch, M, K, plan.p.gamma,
                                       plan.p.gamma_size, plan.p.eps, ctx->act_scratch,
                                       ctx->stream);
    if (e != hipSuccess) return hip_fail(e, op, "rmsnorm pre-pass launch");
    for (int i = 0; i < p.nmat; ++i) p.mat[i].x = ctx->act_scratch;
  }
  // split K: the partial planes (sized for the largest row block) and, after
  // each kernel launch, the fix-up that sums them and runs the epilogue
  const bool split = plan.sk_chunks > 1;
  const int q8_scale = plan.fmt == kQ8;
  const int sf16 = (p.flags & kFlagScaleF16) != 0;
  if (split) {
    QmvParams q = p;
    q.m = plan.kind == kPlanGemm || M < plan.mblock ? M : plan.mblock;
    const long long need = (long long)plan.sk_chunks * splitk_layout(q, plan.sk_nw);
    aexq_status st = grow_scratch(ctx, (void**)&ctx->sk_part, &ctx->sk_cap,
                                  need * (long long)sizeof(float), op, "split-K partial planes");
    if (st) return st;
    p.sk_part = ctx->sk_part;
    p.sk_chunks = plan.sk_chunks;
    p.sk_cs = plan.sk_cs;
  }
  if (plan.kind == kPlanGemm) {
    if (split) splitk_layout(p, plan.sk_nw);
    hipError_t e = qgemm_launch(plan.gentry, p, ctx->stream);
    if (e != hipSuccess) return hip_fail(e, op, "gemm kernel launch");
    if (split) {
      e = splitk_reduce_launch(p, plan.sk_nw, q8_scale, sf16, ctx->stream);
      if (e != hipSuccess) return hip_fail(e, op, "split-K fix-up launch");
    }
    return AEXQ_OK;
  }
  const int ysz = plan.ysz;
  for (int m0 = 0; m0 < M; m0 += plan.mblock) {
    QmvParams q = p;
    q.m = M - m0 < plan.mblock ? M - m0 : plan.mblock;
    q.m_base = m0;
    for (int i = 0; i < q.nmat; ++i) {
      QmvMat& mt = q.mat[i];
      mt.x = (const char*)mt.x + (long long)m0 * q.x_rstride * 2;
      // a head-packed output indexes rows from the tensor's first (out_index)
      if (mt.y && mt.y_hd == 0) mt.y = (char*)mt.y + (long long)m0 * mt.y_rstride * ysz;
      if (mt.res) mt.res = (const char*)mt.res + (long long)m0 * q.r_rstride * ysz;
    }
    if (split) splitk_layout(q, plan.sk_nw);
    hipError_t e = qmm_launch(plan.mentry, q, plan.grid, ctx->stream);
    if (e != hipSuccess) return hip_fail(e, op, "mfma kernel launch");
    if (split) {
      e = splitk_reduce_launch(q, plan.sk_nw, q8_scale, sf16, ctx->stream);
      if (e != hipSuccess) return hip_fail(e, op, "split-K fix-up launch");
    }
  }
  return AEXQ_OK;
}

// Head-packed x: gather it into dense rows in the context's scratch and point
// the plan's activations there.
static aexq_status gather_x(aexq_ctx* ctx, Plan& plan, const char* op) {
  const int width = plan.xg_heads * plan.xg_hd;
  const long long need =
      (long long)plan.xg_batch * plan.xg_rows * width * (plan.xg_f32 ? 4 : 2);
  aexq_status st = grow_scratch(ctx, &ctx->gather_scratch, &ctx->gather_cap, need, op,
                                "head-packed x rows");
  if (st) return st;
  hipError_t e = head_gather_launch(plan.xg_src, plan.xg_f32, plan.xg_rows, plan.xg_heads,
                                    plan.xg_hd, plan.xg_batch, plan.xg_bstride,
                                    ctx->gather_scratch, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, op, "head-packed x gather launch");
  for (int i = 0; i < plan.p.nmat; ++i) plan.p.mat[i].x = ctx->gather_scratch;
  return AEXQ_OK;
}

static aexq_status launch_plan(aexq_ctx* ctx, Plan& plan, const char* op) {
  HIP_TRY(op, hipSetDevice(ctx->device));
  if (plan.x_gather) {
    aexq_status st = gather_x(ctx, plan, op);
    if (st) return st;
  }
  if (plan.kind == kPlanMfma || plan.kind == kPlanGemm) return launch_mfma(ctx, plan, op);
  hipError_t e = plan.fast ? qmv_launch(plan.entry, plan.p, plan.grid, ctx->stream)
                           : generic_launch(plan.fmt, plan.p, plan.grid, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, op, "kernel launch");
  return AEXQ_OK;
}

extern "C" aexq_status aexq_plan_check(aexq_ctx* ctx, const aexq_weight* w, const aexq_tensor* x,
                                       const aexq_tensor* y, const aexq_linear_args* args,
                                       char* diag, size_t diag_len) {
  Plan plan;
  const aexq_weight* ws[1] = {w};
  const aexq_tensor* ys[1] = {y};
  aexq_status st = make_plan(ctx, 1, ws, x, ys, args, false, &plan);
  if (diag && diag_len) {
    if (st)
      snprintf(diag, diag_len, "%s", g_last_error.c_str());
    else if (plan.kind == kPlanGemm)
      snprintf(diag, diag_len,
               "kernel=qgemm bits=%d bm=%d swiglu=%d direct=%d fp16_dequant=%d rms_prepass=%d "
               "tiles=%d grid=%d splitk=%d kstep=%d",
               w->bits, plan.gentry->cfg.bm, (int)plan.gentry->cfg.pair,
               (int)plan.gentry->cfg.direct, (int)plan.gentry->cfg.fd, (int)plan.rms_prepass,
               plan.p.total_tiles, plan.grid, plan.sk_chunks, plan.gentry->cfg.k128 ? 128 : 64);
    else if (plan.kind == kPlanMfma)
      snprintf(diag, diag_len, "kernel=qmm bits=%d mt=%d nt=%d swiglu=%d wide=%d rms_prepass=%d "
               "tiles=%d grid=%d mblock=%d splitk=%d",
               w->bits, plan.mentry->cfg.mt, plan.mentry->cfg.nt, (int)plan.mentry->cfg.pair,
               (int)plan.mentry->cfg.wide, (int)plan.rms_prepass, plan.p.total_tiles, plan.grid,
               plan.mblock, plan.sk_chunks);
    else
      snprintf(diag, diag_len,
               "kernel=%s bits=%d lpr=%d cpl=%d u=%d mmax=%d swiglu=%d tiles=%d grid=%d",
               plan.fast ? "qmv" : "generic", w->bits, plan.fast ? plan.entry->cfg.lpr : 0,
               plan.fast ? plan.entry->cfg.cpl : 0, plan.fast ? plan.entry->cfg.u : 0,
               plan.fast ? plan.entry->cfg.mmax : 0, plan.fast ? (int)plan.entry->cfg.pair : 0,
               plan.p.total_tiles, plan.grid);
  }
  return st;
}

extern "C" aexq_status aexq_linear(aexq_ctx* ctx, const aexq_weight* w, const aexq_tensor* x,
                                   const aexq_tensor* y, const aexq_linear_args* args) {
  Plan plan;
  const aexq_weight* ws[1] = {w};
  const aexq_tensor* ys[1] = {y};
  aexq_status st = make_plan(ctx, 1, ws, x, ys, args, false, &plan);
  if (st) return st;
  return launch_plan(ctx, plan, kLinearOp);
}

extern "C" aexq_status aexq_linear_group(aexq_ctx* ctx, int count, const aexq_weight* const* w,
                                         const aexq_tensor* x, const aexq_tensor* const* y,
                                         const aexq_linear_args* args) {
  if (!w || !y) return fail(AEXQ_ERR_INVALID_ARGUMENT, "aexq_linear_group", "NULL arrays");
  Plan plan;
  aexq_status st = make_plan(ctx, count, w, x, y, args, false, &plan);
  if (st) return st;
  return launch_plan(ctx, plan, "aexq_linear_group");
}

// Where an argmax launch writes its tagged partials: the context's growing
// scratch, or a fixed buffer of `cap` words per plane.
struct Partials {
  unsigned long long* tagged = nullptr;  // three planes of `plane` words
  long long plane = 0;
  unsigned* epoch = nullptr;
  long long cap = 0;
};

// The context's tagged partials for `need` (workgroup, row) entries.
static aexq_status context_partials(aexq_ctx* ctx, long long need, const char* op, Partials* pt) {
  aexq_status st = grow_scratch(ctx, (void**)&ctx->am_tagged, &ctx->am_tagged_cap,
                                3 * need * (long long)sizeof(unsigned long long), op,
                                "tagged argmax partials", true);
  if (!st)
    st = grow_scratch(ctx, (void**)&ctx->am_epoch, &ctx->am_epoch_cap,
                      kArgEpochInts * (long long)sizeof(unsigned), op, "argmax epoch", true);
  if (st) return st;
  pt->tagged = ctx->am_tagged;
  pt->plane = ctx->am_tagged_cap / (3 * (long long)sizeof(unsigned long long));
  pt->epoch = ctx->am_epoch;
  pt->cap = pt->plane;
  return AEXQ_OK;
}

static void bind_partials(QmvParams& p, const Partials& pt, int32_t* argmax, float* gap) {
  p.am_tagged = pt.tagged;
  p.am_plane = pt.plane;
  p.am_epoch = pt.epoch;
  p.am_out = argmax;
  p.am_gap = gap;
}

// The argmax (and top-2 gap) of M logits rows in one launch per block of
// kArgMergeRows rows.  mode: kLogitsF32, kLogitsF16 (fp16 logits),
// kLogitsF32AsF16 (fp32 logits compared after rounding to fp16).  About one
// workgroup per CU in all, at least 1024 columns each; 16-byte loads where
// the rows allow.  AEXQ_ARGMAX_WG_PER_CU overrides the workgroup count (tuning).
static aexq_status argmax_over_logits(aexq_ctx* ctx, const void* logits, int mode, int m, int n,
                                      long long rstride, int32_t* argmax, float* gap,
                                      const char* op) {
  const int esz = mode == kLogitsF16 ? 2 : 4;
  const int vec = 16 / esz;
  const bool vec_ok = ((uintptr_t)logits % 16) == 0 && (rstride * esz) % 16 == 0;
  long long per_cu = 1;
  const char* env = getenv("AEXQ_ARGMAX_WG_PER_CU");
  if (env && atoi(env) > 0) per_cu = atoi(env);
  for (int m0 = 0; m0 < m; m0 += kArgMergeRows) {
    const int mb = m - m0 < kArgMergeRows ? m - m0 : kArgMergeRows;
    long long parts = (per_cu * ctx->cus + mb - 1) / mb;
    const long long most = (n + 1023) / 1024;
    if (parts > most) parts = most;
    if (parts < 1) parts = 1;
    int cols = (int)((n + parts - 1) / parts);
    if (vec_ok) cols = (cols + vec - 1) / vec * vec;
    parts = (n + cols - 1) / cols;
    Partials pt;
    aexq_status st = context_partials(ctx, parts * mb, op, &pt);
    if (st) return st;
    QmvParams p{};
    p.m = mb;
    p.parts = (int)parts;
    bind_partials(p, pt, argmax + m0, gap ? gap + m0 : nullptr);
    hipError_t e = logits_argmax_launch((const char*)logits + (long long)m0 * rstride * esz, mode,
                                        n, rstride, cols, vec_ok ? vec : 1, p, ctx->stream);
    if (e != hipSuccess) return hip_fail(e, op, "argmax launch");
  }
  return AEXQ_OK;
}

static bool lmhead_fused(const Plan& plan) {
  return (plan.fast && plan.entry->cfg.argmax) ||
         (plan.kind == kPlanMfma && plan.mentry->cfg.argmax);
}

// The LM head with the argmax fused into the matvec: M = 1..8 on the
// streaming kernel, M >= 2 on the wide MFMA kernel (one launch per block of up
// to 32 rows); one (best, index, second) partial per workgroup and row, merged
// in the same launch by its last workgroup.  `fixed` null: the partials go to
// the context's scratch (grown as needed).
static aexq_status lmhead_fused_launch(aexq_ctx* ctx, Plan& plan, const char* op,
                                       int32_t* argmax, float* top2_gap, const Partials* fixed) {
  const int M = plan.p.m;
  // the wide kernel runs its tiles on any grid: within a fixed scratch it
  // takes fewer workgroups rather than refuse
  if (fixed && plan.kind == kPlanMfma && (long long)plan.grid * M + 32LL * M > fixed->cap) {
    const long long fit = fixed->cap / M - 32;
    if (fit >= 1 && fit < plan.grid) plan.grid = (int)fit;
  }
  const int grid = plan.grid;  // one partial per workgroup and row
  // a grid of more than 512 workgroups merges in two levels: runs of G = 2^g
  // >= 32 workgroups, at most 31 run mergers (fewer than one XCD's resident
  // workgroups even at one per CU), each polling one round of partials;
  // AEXQ_ARGMAX_ONE_LEVEL keeps the single merge
  int group = 0;
  if (grid > 512 && getenv("AEXQ_ARGMAX_ONE_LEVEL") == nullptr)
    for (group = 5; (grid - 1) >> group > 31;) ++group;
  const int parts = grid + (group ? (grid - 1) >> group : 0);  // and a group partial per run
  const long long need = (long long)parts * M;
  // the MFMA path launches once per block of mblock rows, each merging its own
  const int rows = plan.kind == kPlanMfma && plan.mblock < M ? plan.mblock : M;
  if (rows > kArgMergeRows)
    return fail(AEXQ_ERR_UNSUPPORTED, op, "fused argmax over %d rows per launch (at most %d)",
                rows, kArgMergeRows);
  Partials pt;
  if (fixed) {
    if (need > fixed->cap)
      return fail(AEXQ_ERR_UNSUPPORTED, op,
                  "%d partials a row (one per workgroup and merged run) x %d rows = %lld exceed the fixed scratch of "
                  "%lld | rejectedFallback=allocation",
                  parts, M, need, fixed->cap);
    pt = *fixed;
  } else {
    aexq_status st = context_partials(ctx, need, op, &pt);
    if (st) return st;
  }
  plan.p.parts = parts;
  bind_partials(plan.p, pt, argmax, top2_gap);
  plan.p.am_group = group;
  if (plan.fast) {
    hipError_t e = qmv_launch(plan.entry, plan.p, plan.grid, ctx->stream);
    if (e != hipSuccess) return hip_fail(e, op, "lm head launch");
    return AEXQ_OK;
  }
  return launch_plan(ctx, plan, op);
}

static aexq_status lmhead_argmax(aexq_ctx* ctx, const aexq_weight* w, const aexq_tensor* x,
                                 const aexq_tensor* logits, const aexq_linear_args* args,
                                 int32_t* argmax, float* top2_gap, const char* op) {
  if (!argmax) return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "argmax is NULL");
  if (w && w->batch != 1) return fail(AEXQ_ERR_UNSUPPORTED, op, "stacked LM head");
  Plan plan;
  const aexq_weight* ws[1] = {w};
  const aexq_tensor* ys[1] = {logits};
  aexq_status st = make_plan(ctx, 1, ws, x, ys, args, true, &plan);
  if (st) return st;
  HIP_TRY(op, hipSetDevice(ctx->device));
  if (lmhead_fused(plan)) return lmhead_fused_launch(ctx, plan, op, argmax, top2_gap, nullptr);
  // logits first (into the caller's tensor or a scratch buffer), then the argmax pass
  const int M = plan.p.m;
  void* lg = nullptr;
  long long rstride = plan.p.mat[0].y_rstride;
  const bool f16_cmp = (plan.p.flags & kFlagArgF16) != 0;
  int mode = f16_cmp ? kLogitsF32AsF16 : kLogitsF32;
  if (logits) {
    lg = logits->data;
    if (logits->dtype == AEXQ_DTYPE_F16) mode = kLogitsF16;
  } else {
    const long long need = (long long)M * w->n;
    st = grow_scratch(ctx, (void**)&ctx->logits_scratch, &ctx->logits_cap,
                      need * (long long)sizeof(float), op, "logits");
    if (st) return st;
    lg = ctx->logits_scratch;
    plan.p.mat[0].y = lg;
    plan.p.mat[0].y_rstride = w->n;
    plan.p.flags |= kFlagYf32;
    rstride = w->n;
  }
  st = launch_plan(ctx, plan, op);
  if (st) return st;
  return argmax_over_logits(ctx, lg, mode, M, w->n, rstride, argmax, top2_gap, op);
}

extern "C" aexq_status aexq_lmhead_argmax(aexq_ctx* ctx, const aexq_weight* w,
                                          const aexq_tensor* x, const aexq_tensor* logits,
                                          int32_t* argmax, float* top2_gap) {
  return lmhead_argmax(ctx, w, x, logits, nullptr, argmax, top2_gap, "aexq_lmhead_argmax");
}

extern "C" aexq_status aexq_lmhead_argmax_ex(aexq_ctx* ctx, const aexq_weight* w,
                                             const aexq_tensor* x, const aexq_tensor* logits,
                                             const aexq_linear_args* args, int32_t* argmax,
                                             float* top2_gap) {
  const char* op = "aexq_lmhead_argmax_ex";
  if (args && (args->flags & ~(unsigned)(AEXQ_EPI_RMSNORM_IN | AEXQ_EPI_ARGMAX_F16)))
    return fail(AEXQ_ERR_UNSUPPORTED, op,
                "epilogue flags 0x%x: the LM head takes RMSNorm-in and the fp16-logit argmax only "
                "| rejectedFallback=epilogue",
                args->flags);
  return lmhead_argmax(ctx, w, x, logits, args, argmax, top2_gap, op);
}

extern "C" aexq_status aexq_lmhead_argmax_noalloc(aexq_ctx* ctx, const aexq_weight* w,
                                                  const aexq_tensor* x, int32_t* argmax,
                                                  float* top2_gap) {
  const char* op = "aexq_lmhead_argmax_noalloc";
  if (!argmax) return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "argmax is NULL");
  if (w && w->batch != 1) return fail(AEXQ_ERR_UNSUPPORTED, op, "stacked LM head");
  Plan plan;
  const aexq_weight* ws[1] = {w};
  const aexq_tensor* ys[1] = {nullptr};
  aexq_status st = make_plan(ctx, 1, ws, x, ys, nullptr, true, &plan);
  if (st) return st;
  if (!lmhead_fused(plan))
    return fail(AEXQ_ERR_UNSUPPORTED, op,
                "no fused-argmax kernel for M=%d K=%d (the logits pass needs a buffer of its "
                "own) | rejectedFallback=allocation",
                plan.p.m, plan.p.k);
  if (!ctx->noalloc)
    return fail(AEXQ_ERR_DEVICE, op, "no device address for the fixed scratch on device %d | hip=%s",
                ctx->device,
                hipGetErrorString(ctx->device >= 0 && ctx->device < kMaxDevices
                                      ? g_noalloc_err[ctx->device]
                                      : hipErrorInvalidDevice));
  HIP_TRY(op, hipSetDevice(ctx->device));
  Partials fixed;
  fixed.tagged = ctx->noalloc;
  fixed.plane = kNoAllocParts;
  fixed.epoch = (unsigned*)(ctx->noalloc + 3 * kNoAllocParts);
  fixed.cap = kNoAllocParts;
  return lmhead_fused_launch(ctx, plan, op, argmax, top2_gap, &fixed);
}

extern "C" aexq_status aexq_argmax(aexq_ctx* ctx, const aexq_tensor* logits, int32_t* argmax,
                                   float* top2_gap) {
  const char* op = "aexq_argmax";
  if (!ctx || !argmax) return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "NULL argument");
  TensorView v;
  aexq_status st = view_tensor(logits, op, "logits", &v);
  if (st) return st;
  if (v.head_dim)
    return fail(AEXQ_ERR_UNSUPPORTED, op, "head-packed logits | rejectedFallback=layout");
  HIP_TRY(op, hipSetDevice(ctx->device));
  return argmax_over_logits(ctx, v.data, v.dtype == AEXQ_DTYPE_F16 ? kLogitsF16 : kLogitsF32,
                            v.rows, v.width, v.rstride, argmax, top2_gap, op);
}

extern "C" aexq_status aexq_dequant(aexq_ctx* ctx, const aexq_weight* w, float* out) {
  const char* op = "aexq_dequant";
  if (!ctx || !w || !out) return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "NULL argument");
  if (w->device != ctx->device)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "weight on device %d, context on device %d",
                w->device, ctx->device);
  HIP_TRY(op, hipSetDevice(ctx->device));
  const int fmt = w->bits == 8 ? kQ8 : kQ4;
  hipError_t e = dequant_launch(fmt, w->codes, w->scales, w->scale_dtype == AEXQ_DTYPE_F16, w->n,
                                w->k, w->block, out, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, op, "dequant launch");
  return AEXQ_OK;
}

// ---------------------------------------------------------------------------
// decode-step operators
// ---------------------------------------------------------------------------
extern "C" aexq_status aexq_rmsnorm(aexq_ctx* ctx, const aexq_tensor* x, const aexq_tensor* y,
                                    const float* gamma, int gamma_size, float eps) {
  const char* op = "aexq_rmsnorm";
  if (!ctx) return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "ctx is NULL");
  TensorView xv, yv;
  aexq_status st = view_tensor(x, op, "x", &xv);
  if (st) return st;
  st = view_tensor(y, op, "y", &yv);
  if (st) return st;
  if (yv.rows != xv.rows || yv.width != xv.width)
    return fail(AEXQ_ERR_SHAPE, op, "y [%d][%d] != x [%d][%d] | layer=RMSNorm", yv.rows, yv.width,
                xv.rows, xv.width);
  if (yv.dtype != AEXQ_DTYPE_F16 || yv.rstride != yv.width)
    return fail(AEXQ_ERR_UNSUPPORTED, op,
                "y must be fp16 rows of exactly W elements | layer=RMSNorm | rejectedFallback=layout");
  if (xv.batch != yv.batch || (yv.batch > 1 && yv.bstride != (long long)yv.rows * yv.width))
    return fail(AEXQ_ERR_SHAPE, op, "batched y must be contiguous [batch][rows][W]");
  if (gamma && gamma_size <= 0)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "gamma_size=%d", gamma_size);
  HIP_TRY(op, hipSetDevice(ctx->device));
  hipError_t e = rmsnorm_rows_launch(xv.data, xv.dtype == AEXQ_DTYPE_F32, xv.rstride,
                                     xv.batch == 1 ? 0 : xv.bstride, xv.batch, xv.rows, xv.width,
                                     gamma, gamma_size, eps, yv.data, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, op, "rmsnorm launch");
  return AEXQ_OK;
}

extern "C" aexq_status aexq_embed_q8(aexq_ctx* ctx, const aexq_weight* table,
                                     const int32_t* tokens, int m, void* out) {
  const char* op = "aexq_embed_q8";
  if (!ctx || !table || !tokens || !out) return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "NULL argument");
  if (table->device != ctx->device)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "table on device %d, context on device %d",
                table->device, ctx->device);
  if (table->bits != 8 || table->block != table->k)
    return fail(AEXQ_ERR_UNSUPPORTED, op, "embedding table must be Q8 with one scale per row");
  if (m <= 0) return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "m=%d", m);
  HIP_TRY(op, hipSetDevice(ctx->device));
  hipError_t e = embed_q8_launch(table->codes, table->scales, table->scale_dtype == AEXQ_DTYPE_F16,
                                 table->k, tokens, m, table->n, out, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, op, "embedding launch");
  return AEXQ_OK;
}

extern "C" aexq_status aexq_rope_kv_append(aexq_ctx* ctx, void* q, const void* k, const void* v,
                                           void* k_cache, void* v_cache, int heads_q,
                                           int heads_kv, int head_dim, int capacity, int position,
                                           const float* cos_table, const float* sin_table) {
  const char* op = "aexq_rope_kv_append";
  if (!ctx || !q || !k || !v || !k_cache || !v_cache || !cos_table || !sin_table)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "NULL argument");
  if (heads_q <= 0 || heads_kv <= 0 || head_dim <= 0 || (head_dim & 1))
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "heads_q=%d heads_kv=%d head_dim=%d", heads_q,
                heads_kv, head_dim);
  if (position < 0 || position >= capacity)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "position=%d outside the cache capacity %d",
                position, capacity);
  HIP_TRY(op, hipSetDevice(ctx->device));
  hipError_t e = rope_kv_launch(q, k, v, k_cache, v_cache, heads_q, heads_kv, head_dim, capacity,
                                position, cos_table, sin_table, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, op, "rope launch");
  return AEXQ_OK;
}

// Shared checks of the decode attention entry points; sizes the split scratch.
static aexq_status attn_prepare(aexq_ctx* ctx, const char* op, int heads_q, int heads_kv,
                                int head_dim, int capacity, int length) {
  if (head_dim != 128)
    return fail(AEXQ_ERR_UNSUPPORTED, op, "head_dim=%d (kernel is built for 128) | layer=SDPA",
                head_dim);
  if (heads_kv <= 0 || heads_q <= 0 || heads_q % heads_kv != 0)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "heads_q=%d heads_kv=%d", heads_q, heads_kv);
  const int group = heads_q / heads_kv;
  if (group != 1 && group != 2 && group != 4 && group != 8)
    return fail(AEXQ_ERR_UNSUPPORTED, op, "query heads per key head = %d (1, 2, 4 or 8)", group);
  if (length <= 0 || length > capacity)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "length=%d capacity=%d", length, capacity);
  const int splits = attn_splits(length);
  if (splits > attn_max_splits())
    return fail(AEXQ_ERR_UNSUPPORTED, op, "length=%d needs %d splits (at most %d)", length,
                splits, attn_max_splits());
  const long long need = (long long)heads_q * splits * attn_part_stride();
  HIP_TRY(op, hipSetDevice(ctx->device));
  aexq_status st = grow_scratch(ctx, (void**)&ctx->attn_part, &ctx->attn_cap,
                                need * (long long)sizeof(float), op, "attention split partials");
  if (st) return st;
  // split counters start at zero; every launch leaves them at zero
  return grow_scratch(ctx, (void**)&ctx->attn_count, &ctx->attn_count_cap,
                      (long long)heads_kv * attn_counter_stride() * (long long)sizeof(int), op,
                      "attention split counters", true);
}

extern "C" aexq_status aexq_attention_decode(aexq_ctx* ctx, const void* q, const void* k_cache,
                                             const void* v_cache, int heads_q, int heads_kv,
                                             int head_dim, int capacity, int length, float scale,
                                             void* out) {
  const char* op = "aexq_attention_decode";
  if (!ctx || !q || !k_cache || !v_cache || !out)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "NULL argument");
  aexq_status st = attn_prepare(ctx, op, heads_q, heads_kv, head_dim, capacity, length);
  if (st) return st;
  hipError_t e = attn_decode_launch(q, k_cache, v_cache, heads_q, heads_kv, capacity, length,
                                    scale, ctx->attn_part, ctx->attn_count, out, nullptr, nullptr,
                                    nullptr, nullptr, nullptr, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, op, "attention launch");
  return AEXQ_OK;
}

extern "C" aexq_status aexq_attention_decode_rope(aexq_ctx* ctx, const void* q, const void* k,
                                                  const void* v, void* k_cache, void* v_cache,
                                                  int heads_q, int heads_kv, int head_dim,
                                                  int capacity, int length, const float* cos_table,
                                                  const float* sin_table, float scale, void* out) {
  const char* op = "aexq_attention_decode_rope";
  if (!ctx || !q || !k || !v || !k_cache || !v_cache || !cos_table || !sin_table || !out)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "NULL argument");
  aexq_status st = attn_prepare(ctx, op, heads_q, heads_kv, head_dim, capacity, length);
  if (st) return st;
  hipError_t e = attn_decode_launch(q, k_cache, v_cache, heads_q, heads_kv, capacity, length,
                                    scale, ctx->attn_part, ctx->attn_count, out, k, v, cos_table,
                                    sin_table, nullptr, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, op, "attention launch");
  return AEXQ_OK;
}

extern "C" aexq_status aexq_attention_decode_rope_at(aexq_ctx* ctx, const void* q, const void* k,
                                                     const void* v, void* k_cache, void* v_cache,
                                                     int heads_q, int heads_kv, int head_dim,
                                                     int capacity, const int32_t* position,
                                                     const float* cos_table,
                                                     const float* sin_table, float scale,
                                                     void* out) {
  const char* op = "aexq_attention_decode_rope_at";
  if (!ctx || !q || !k || !v || !k_cache || !v_cache || !position || !cos_table || !sin_table ||
      !out)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "NULL argument");
  // sized for the whole cache: the launch covers every position the device
  // counter may name
  aexq_status st = attn_prepare(ctx, op, heads_q, heads_kv, head_dim, capacity, capacity);
  if (st) return st;
  hipError_t e = attn_decode_launch(q, k_cache, v_cache, heads_q, heads_kv, capacity, capacity,
                                    scale, ctx->attn_part, ctx->attn_count, out, k, v, cos_table,
                                    sin_table, position, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, op, "attention launch");
  return AEXQ_OK;
}

extern "C" aexq_status aexq_decode_advance(aexq_ctx* ctx, int32_t* position, int32_t* token,
                                           const int32_t* argmax, int32_t* tokens_out,
                                           int tokens_cap) {
  const char* op = "aexq_decode_advance";
  if (!ctx || !position || !token || !argmax)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "NULL argument");
  if (tokens_out && tokens_cap <= 0)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "tokens_cap=%d", tokens_cap);
  HIP_TRY(op, hipSetDevice(ctx->device));
  hipError_t e = decode_advance_launch(position, token, argmax, tokens_out,
                                       tokens_out ? tokens_cap : 0, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, op, "advance launch");
  return AEXQ_OK;
}

// ---------------------------------------------------------------------------
// The decoder layers of a decode step as one persistent launch
// (DecodeCore, DEC:463-585; the per-layer loop LF:996-1136).  The decoder
// object holds the layers' device pointers and the tagged exchange buffers;
// aexq_decoder_run allocates nothing, so a graph may capture it.
// ---------------------------------------------------------------------------
struct aexq_decoder {
  aexq_ctx* ctx = nullptr;
  int device = 0;
  int grid = 0;
  StepParams p{};
  void* mem = nullptr;  // layer table + exchange buffers
};

// Workgroups of the fused step: 128 (one per CU on half of the part) when the
// cache fits their attention splits, else 256.
static int decoder_grid(int hkv, int cap, int requested) {
  if (requested > 0) return requested;
  for (int g = 128; g <= 256; g *= 2) {
    int s = g / hkv;
    if (s > kStepMaxSplits) s = kStepMaxSplits;
    if (s > 0 && (long long)s * kStepMaxSplitPos >= cap) return g;
  }
  return 256;
}

extern "C" aexq_status aexq_decoder_create(aexq_ctx* ctx, const aexq_decoder_config* cfg,
                                           const aexq_decoder_layer* layers, int count,
                                           const aexq_weight* embedding, aexq_decoder** out) {
  const char* op = "aexq_decoder_create";
  if (!ctx || !cfg || !layers || !embedding || !out)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "NULL argument");
  if (count <= 0) return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "count=%d", count);
  if (count > kStepMaxLayers)
    return fail(AEXQ_ERR_UNSUPPORTED, op, "%d layers (the fused step stages at most %d layer "
                "entries in LDS) | rejectedFallback=per-operator step", count, kStepMaxLayers);
  if (!cfg->rope_cos || !cfg->rope_sin)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "rope tables are NULL");
  const int hq = cfg->heads_q, hkv = cfg->heads_kv, cap = cfg->capacity;
  if (cfg->head_dim != kStepHeadDim)
    return fail(AEXQ_ERR_UNSUPPORTED, op, "head_dim=%d (the fused step takes %d) | "
                "rejectedFallback=per-operator step", cfg->head_dim, kStepHeadDim);
  if (hq <= 0 || hkv <= 0 || hq % hkv != 0 || cap <= 0)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "heads_q=%d heads_kv=%d capacity=%d", hq, hkv,
                cap);
  const aexq_weight* l0q = layers[0].q_proj;
  if (!l0q) return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "layer 0 q_proj is NULL");
  const int hid = l0q->k, qw = hq * kStepHeadDim, kvw = hkv * kStepHeadDim;
  const int inter = layers[0].gate_proj ? layers[0].gate_proj->n : 0;
  const int sdt = l0q->scale_dtype;
  // the layer format of q_proj: Q4 with one scale per 32 or 16 codes, or Q8
  // with one scale per row; every weight of every layer must share it
  const int fmt = l0q->bits == 8 ? kQ8 : kQ4;
  const int gmode = fmt == kQ8 ? kGRow : (l0q->block == 16 ? kG16 : kG32);
  const bool fmt_ok = fmt == kQ8 ? l0q->block == l0q->k : (l0q->block == 16 || l0q->block == 32);
  if (!fmt_ok)
    return fail(AEXQ_ERR_UNSUPPORTED, op,
                "layer 0 q_proj: bits=%d block=%d (the fused step takes Q4 with one scale per 32 "
                "or 16 codes, or Q8 with one scale per row) | rejectedFallback=per-operator step",
                l0q->bits, l0q->block);
  for (int l = 0; l < count; ++l) {
    const aexq_decoder_layer& L = layers[l];
    const aexq_weight* ws[7] = {L.q_proj, L.k_proj, L.v_proj, L.o_proj, L.gate_proj, L.up_proj,
                                L.down_proj};
    const int nn[7] = {qw, kvw, kvw, hid, inter, inter, hid};
    const int kk[7] = {hid, hid, hid, qw, hid, hid, inter};
    for (int i = 0; i < 7; ++i) {
      const aexq_weight* w = ws[i];
      if (!w) return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "layer %d weight %d is NULL", l, i);
      if (w->n != nn[i] || w->k != kk[i])
        return fail(AEXQ_ERR_SHAPE, op, "layer %d weight %d is %dx%d, expected %dx%d", l, i,
                    w->n, w->k, nn[i], kk[i]);
      const int want_block = fmt == kQ8 ? w->k : l0q->block;
      if (w->bits != l0q->bits || w->block != want_block || w->batch != 1 ||
          w->scale_dtype != sdt)
        return fail(AEXQ_ERR_UNSUPPORTED, op,
                    "layer %d weight %d: bits=%d block=%d batch=%d scale_dtype=%d, layer 0 q_proj "
                    "bits=%d block=%d scale_dtype=%d (the fused step takes one unstacked format "
                    "for every weight) | rejectedFallback=per-operator step", l, i, w->bits,
                    w->block, w->batch, w->scale_dtype, l0q->bits, l0q->block, sdt);
      if (w->device != ctx->device)
        return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "layer %d weight %d lives on device %d", l, i,
                    w->device);
    }
    if (!L.attn_norm || !L.mlp_norm || !L.k_cache || !L.v_cache)
      return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "layer %d: NULL norm or cache", l);
  }
  if (embedding->bits != 8 || embedding->k != hid || embedding->batch != 1)
    return fail(AEXQ_ERR_UNSUPPORTED, op, "embedding bits=%d k=%d batch=%d (Q8 of width %d)",
                embedding->bits, embedding->k, embedding->batch, hid);
  const int ce = fmt == kQ8 ? 16 : 32;  // codes per 16-byte chunk
  if (hid % 32 || hid > kStepMaxHidden || inter % 32 || inter > kStepMaxInter ||
      !decode_layers_supported(fmt, gmode, hq / hkv, hid / ce, qw / ce, inter / ce))
    return fail(AEXQ_ERR_UNSUPPORTED, op,
                "hidden=%d q width=%d intermediate=%d, %d q heads per kv head, %s: no fused-step "
                "kernel for these shapes | rejectedFallback=per-operator step",
                hid, qw, inter, hq / hkv, fmt == kQ8 ? "Q8" : "Q4");
  const int grid = decoder_grid(hkv, cap, cfg->workgroups);
  int splits = grid / hkv;
  if (splits > kStepMaxSplits) splits = kStepMaxSplits;
  const int sp = (int)round_up((cap + splits - 1) / splits, 8);
  const int merge = hq * kStepHeadDim / grid;
  const int rq = (int)round_up((qw + 2 * kvw + grid - 1) / grid, 4);
  const int rh = (int)round_up((hid + grid - 1) / grid, 2);
  const int ri = (int)round_up((inter + grid - 1) / grid, 4);
  if (grid < hkv || splits < 1 || sp > kStepMaxSplitPos || merge < 1 || merge > kStepMaxMerge ||
      kStepHeadDim % merge || merge * grid != hq * kStepHeadDim || merge % 8 ||
      splits * (merge / 8) > 64 || rq > 4 * kStepComputeWaves || rh > kStepComputeWaves ||
      ri > 4 * kStepComputeWaves || rq > kStepOutWords || ri > kStepOutWords || rq > 64 ||
      ri > 64 || rh < 1 || merge > 64 || (hq / hkv) * kStepPartStride > kStepOutWords)
    return fail(AEXQ_ERR_UNSUPPORTED, op,
                "capacity=%d on %d workgroups: %d splits of %d positions, %d merged dims, rows "
                "%d/%d/%d per workgroup | rejectedFallback=per-operator step",
                cap, grid, splits, sp, merge, rq, rh, ri);
  HIP_TRY(op, hipSetDevice(ctx->device));
  int per_cu = 0;
  HIP_TRY(op, decode_layers_occupancy(fmt, gmode, &per_cu));
  if ((long long)per_cu * ctx->cus < grid)
    return fail(AEXQ_ERR_UNSUPPORTED, op,
                "%d workgroups are not co-resident (%d per CU x %d CUs) | rejectedFallback="
                "per-operator step", grid, per_cu, ctx->cus);

  // one allocation: layer table, then the exchange buffers (256-byte aligned)
  std::vector<StepLayer> table((size_t)count);
  for (int l = 0; l < count; ++l) {
    const aexq_decoder_layer& L = layers[l];
    const aexq_weight* ws[7] = {L.q_proj, L.k_proj, L.v_proj, L.o_proj, L.gate_proj, L.up_proj,
                                L.down_proj};
    for (int i = 0; i < 7; ++i) {
      table[l].w[i] = ws[i]->codes;
      table[l].s[i] = ws[i]->scales;
    }
    table[l].g_attn = L.attn_norm;
    table[l].g_mlp = L.mlp_norm;
    table[l].kc = (uint16_t*)L.k_cache;
    table[l].vc = (uint16_t*)L.v_cache;
  }
  // the polled vectors in kStepReplicas copies of whole 4 KB pages each, every
  // buffer on a 4 KB boundary (the allocation is over-sized by a page to align)
  const int rs[8] = {step_replica_stride(hid), step_replica_stride(qw + 2 * kvw), 0,
                     step_replica_stride(qw), step_replica_stride(hid), step_replica_stride(inter),
                     0, 0};
  const long long words[8] = {(long long)kStepReplicas * rs[0], (long long)kStepReplicas * rs[1],
                              (long long)hq * splits * kStepPartStride,
                              (long long)kStepReplicas * rs[3], (long long)kStepReplicas * rs[4],
                              (long long)kStepReplicasH * rs[5], 1, 1};
  long long off[9];
  off[0] = round_up((long long)count * sizeof(StepLayer), 4096);
  for (int i = 0; i < 8; ++i) off[i + 1] = off[i] + round_up(words[i] * 4, 4096);
  aexq_decoder* d = new aexq_decoder();
  hipError_t e = hipMalloc(&d->mem, (size_t)off[8] + 4096);
  if (e == hipSuccess) e = hipMemset(d->mem, 0, (size_t)off[8] + 4096);
  if (e == hipSuccess)
    e = hipMemcpy(d->mem, table.data(), (size_t)count * sizeof(StepLayer), hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(d->mem);
    delete d;
    return hip_fail(e, op, "decoder buffers");
  }
  // the layer table at the allocation's start; the buffers at offsets from its
  // first 4 KB boundary (off[0] >= the table's bytes, so they never overlap it)
  char* const table_at = (char*)d->mem;
  char* const base = (char*)(uintptr_t)round_up((long long)(uintptr_t)table_at, 4096);
  StepParams& p = d->p;
  p.layers = (const StepLayer*)table_at;
  p.nlayers = count;
  p.hidden = hid;
  p.qw = qw;
  p.kvw = kvw;
  p.inter = inter;
  p.hq = hq;
  p.hkv = hkv;
  p.cap = cap;
  p.fmt = fmt;
  p.gmode = gmode;
  p.sf16 = sdt == AEXQ_DTYPE_F16;
  p.eps = cfg->rms_eps;
  p.scale = cfg->attn_scale;
  p.emb_codes = embedding->codes;
  p.emb_scales = embedding->scales;
  p.emb_sf16 = embedding->scale_dtype == AEXQ_DTYPE_F16;
  p.vocab = embedding->n;
  p.cos_t = cfg->rope_cos;
  p.sin_t = cfg->rope_sin;
  p.xa_t = (uint32_t*)(base + off[0]);
  p.qkv_t = (uint32_t*)(base + off[1]);
  p.part_t = (uint32_t*)(base + off[2]);
  p.attn_t = (uint32_t*)(base + off[3]);
  p.xb_t = (uint32_t*)(base + off[4]);
  p.h_t = (uint32_t*)(base + off[5]);
  p.xa_rs = rs[0];
  p.qkv_rs = rs[1];
  p.attn_rs = rs[3];
  p.xb_rs = rs[4];
  p.h_rs = rs[5];
  p.epoch = (uint32_t*)(base + off[6]);
  p.err = (int*)(base + off[7]);
  p.rows_qkv = rq;
  p.rows_hid = rh;
  p.rows_inter = ri;
  p.splits = splits;
  p.split_pos = sp;
  p.merge_dims = merge;
  d->ctx = ctx;
  d->device = ctx->device;
  d->grid = grid;
  *out = d;
  return AEXQ_OK;
}

extern "C" aexq_status aexq_decoder_run(aexq_decoder* d, const int32_t* token,
                                        const int32_t* position, void* hidden_out) {
  const char* op = "aexq_decoder_run";
  if (!d || !token || !position || !hidden_out)
    return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "NULL argument");
  HIP_TRY(op, hipSetDevice(d->device));
  StepParams p = d->p;
  p.token = token;
  p.pos = position;
  p.out = (uint16_t*)hidden_out;
  hipError_t e = decode_layers_launch(p, d->grid, d->ctx->stream);
  if (e != hipSuccess) return hip_fail(e, op, "fused step launch");
  return AEXQ_OK;
}

extern "C" aexq_status aexq_decoder_error(aexq_decoder* d, int* flag) {
  const char* op = "aexq_decoder_error";
  if (!d || !flag) return fail(AEXQ_ERR_INVALID_ARGUMENT, op, "NULL argument");
  HIP_TRY(op, hipSetDevice(d->device));
  HIP_TRY(op, hipStreamSynchronize(d->ctx->stream));
  HIP_TRY(op, hipMemcpy(flag, d->p.err, sizeof(int), hipMemcpyDeviceToHost));
  HIP_TRY(op, hipMemset(d->p.err, 0, sizeof(int)));
  return AEXQ_OK;
}

extern "C" aexq_status aexq_decoder_info(const aexq_decoder* d, int* workgroups, int* splits,
                                         int* split_positions) {
  if (!d) return fail(AEXQ_ERR_INVALID_ARGUMENT, "aexq_decoder_info", "NULL decoder");
  if (workgroups) *workgroups = d->grid;
  if (splits) *splits = d->p.splits;
  if (split_positions) *split_positions = d->p.split_pos;
  return AEXQ_OK;
}

extern "C" void aexq_decoder_release(aexq_decoder* d) {
  if (!d) return;
  (void)hipSetDevice(d->device);
  (void)hipFree(d->mem);
  delete d;
}
