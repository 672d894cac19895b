// P/Invoke surface of libaexq (include/aexq.h), the C ABI of the MI355X
// quantized decode-linear library.  Every entry point the header declares has
// one DllImport here; the structs carry the C compiler's field offsets for
// LP64 (Linux) and LLP64 (Windows) alike, which tests/test_cpu_host.py checks
// against offsetof().  Paths in comments are relative to the reference root.
using System;
using System.Runtime.InteropServices;
using System.Text;

namespace Aexis.Hip
{
    /// <summary>Constants of include/aexq.h.</summary>
    public static class Aexq
    {
        public const int AbiVersion = 1;

        // aexq_status
        public const int Ok = 0;
        public const int ErrInvalidArgument = 1;
        public const int ErrUnsupported = 2;
        public const int ErrShape = 3;
        public const int ErrDevice = 4;
        public const int ErrOutOfMemory = 5;
        public const int ErrFormat = 6;

        // element types of activations, outputs and scales
        public const int DtypeF16 = 1;
        public const int DtypeF32 = 2;

        // Q4 nibble codes (NcnnQ8Archive.WriteQ4 stores q & 0xF: two's complement)
        public const int NibbleTwos = 0;
        public const int NibbleOffset8 = 1;

        // storage layouts (GS:10818-10857; head-packed GL:1003-1043)
        public const int LayoutLinear = 0;
        public const int LayoutPack4Linear = 1;
        public const int LayoutPack4Tiled = 2;
        public const int LayoutHeadPacked = 3;

        // epilogue flags
        public const uint EpiRmsNormIn = 0x1u;
        public const uint EpiSwiGluOut = 0x2u;
        public const uint EpiResidualAdd = 0x4u;
        public const uint EpiArgmaxF16 = 0x8u;    // LM head: argmax over fp16-rounded logits (ARGBHalf)
        public const uint EpiExactDequant = 0x10u; // Q4 at M > 32: float(q) * scale kept exact

        // the texture size limit the storage rules are written against (GS:10852)
        public const int TileWidthLimit = 8192;
    }

    /// <summary>aexq_shape: AexisGraphSession.BufferShape(dims, w, h, d, c).</summary>
    [StructLayout(LayoutKind.Explicit, Size = 20)]
    public struct AexqShape
    {
        [FieldOffset(0)] public int dims;
        [FieldOffset(4)] public int w;
        [FieldOffset(8)] public int h;
        [FieldOffset(12)] public int d;
        [FieldOffset(16)] public int c;

        public AexqShape(int dims, int w, int h, int d, int c)
        {
            this.dims = dims;
            this.w = w;
            this.h = h;
            this.d = d;
            this.c = c;
        }
    }

    /// <summary>aexq_tensor: a device tensor standing in for a Pack4/LinearMat texture.</summary>
    [StructLayout(LayoutKind.Explicit, Size = 72)]
    public struct AexqTensor
    {
        [FieldOffset(0)] public AexqShape logical;
        [FieldOffset(20)] public AexqShape storage;
        [FieldOffset(40)] public int layout;
        [FieldOffset(44)] public int dtype;
        [FieldOffset(48)] public IntPtr data;
        [FieldOffset(56)] public int batch;
        [FieldOffset(64)] public long batchStride;
    }

    /// <summary>aexq_linear_args: ncnn Gemm params 0, 1, 6, 10 and the fused epilogues.</summary>
    [StructLayout(LayoutKind.Explicit, Size = 64)]
    public struct AexqLinearArgs
    {
        [FieldOffset(0)] public float alpha;
        [FieldOffset(4)] public float beta;
        [FieldOffset(8)] public IntPtr c;
        [FieldOffset(16)] public int broadcastC;
        [FieldOffset(24)] public IntPtr rmsGamma;
        [FieldOffset(32)] public int rmsGammaSize;
        [FieldOffset(36)] public float rmsEps;
        [FieldOffset(40)] public IntPtr up;
        [FieldOffset(48)] public IntPtr residual;
        [FieldOffset(56)] public uint flags;

        /// <summary>alpha = beta = 1, no C term, no epilogue (the Gemm defaults, GL:25-26).</summary>
        public static AexqLinearArgs Default()
        {
            return new AexqLinearArgs { alpha = 1f, beta = 1f, broadcastC = -1 };
        }
    }

    /// <summary>aexq_weight_info.</summary>
    [StructLayout(LayoutKind.Explicit, Size = 48)]
    public struct AexqWeightInfo
    {
        [FieldOffset(0)] public int bits;
        [FieldOffset(4)] public int n;
        [FieldOffset(8)] public int k;
        [FieldOffset(12)] public int block;
        [FieldOffset(16)] public int scaleDtype;
        [FieldOffset(20)] public int nibbleCode;
        [FieldOffset(24)] public int batch;
        [FieldOffset(32)] public long codeBytes;
        [FieldOffset(40)] public long scaleBytes;
    }

    /// <summary>aexq_decoder_layer: one layer's weights, norms and caches.</summary>
    [StructLayout(LayoutKind.Explicit, Size = 88)]
    public struct AexqDecoderLayer
    {
        [FieldOffset(0)] public IntPtr qProj;
        [FieldOffset(8)] public IntPtr kProj;
        [FieldOffset(16)] public IntPtr vProj;
        [FieldOffset(24)] public IntPtr oProj;
        [FieldOffset(32)] public IntPtr gateProj;
        [FieldOffset(40)] public IntPtr upProj;
        [FieldOffset(48)] public IntPtr downProj;
        [FieldOffset(56)] public IntPtr attnNorm;
        [FieldOffset(64)] public IntPtr mlpNorm;
        [FieldOffset(72)] public IntPtr kCache;
        [FieldOffset(80)] public IntPtr vCache;
    }

    /// <summary>aexq_decoder_config.</summary>
    [StructLayout(LayoutKind.Explicit, Size = 48)]
    public struct AexqDecoderConfig
    {
        [FieldOffset(0)] public int headsQ;
        [FieldOffset(4)] public int headsKv;
        [FieldOffset(8)] public int headDim;
        [FieldOffset(12)] public int capacity;
        [FieldOffset(16)] public float rmsEps;
        [FieldOffset(20)] public float attnScale;
        [FieldOffset(24)] public IntPtr ropeCos;
        [FieldOffset(32)] public IntPtr ropeSin;
        [FieldOffset(40)] public int workgroups;
    }

    /// <summary>The DllImports of include/aexq.h (one per declared function).</summary>
    public static class Native
    {
        const string Lib = "aexq";   // libaexq.so / aexq.dll beside the backend assembly

        // ---- library / context
        [DllImport(Lib)] public static extern int aexq_abi_version();
        [DllImport(Lib)] public static extern IntPtr aexq_last_error();
        [DllImport(Lib)] public static extern int aexq_create(int device, IntPtr hipStream, out IntPtr ctx);
        [DllImport(Lib)] public static extern void aexq_destroy(IntPtr ctx);
        [DllImport(Lib)] public static extern int aexq_set_stream(IntPtr ctx, IntPtr hipStream);
        [DllImport(Lib)] public static extern int aexq_synchronize(IntPtr ctx);

        // ---- weights (load time); scales are fp32 (the archives' dtype) or fp16 as ushort bits
        [DllImport(Lib)] public static extern int aexq_weight_q8(IntPtr ctx, uint[] packed, float[] scales,
            int scaleDtype, int n, int k, int block, out IntPtr w);
        [DllImport(Lib, EntryPoint = "aexq_weight_q8")] public static extern int aexq_weight_q8_f16(IntPtr ctx,
            uint[] packed, ushort[] scales, int scaleDtype, int n, int k, int block, out IntPtr w);
        [DllImport(Lib)] public static extern int aexq_weight_q4(IntPtr ctx, uint[] packed, float[] scales,
            int scaleDtype, int n, int k, int block, int nibbleCode, out IntPtr w);
        [DllImport(Lib, EntryPoint = "aexq_weight_q4")] public static extern int aexq_weight_q4_f16(IntPtr ctx,
            uint[] packed, ushort[] scales, int scaleDtype, int n, int k, int block, int nibbleCode, out IntPtr w);
        [DllImport(Lib)] public static extern int aexq_weight_q8_from_f32(IntPtr ctx, float[] data, int n, int k,
            int transB, out IntPtr w);
        [DllImport(Lib)] public static extern int aexq_weight_q4_from_f32(IntPtr ctx, float[] data, int n, int k,
            int transB, out IntPtr w);
        [DllImport(Lib)] public static extern int aexq_archive_header(byte[] buf, UIntPtr len, out int quantBits,
            out int defaultBlock, out int recordCount);
        [DllImport(Lib)] public static extern int aexq_weight_from_record(IntPtr ctx, int bits, byte[] record,
            UIntPtr recordLen, int n, int k, out IntPtr w, out UIntPtr consumed);
        [DllImport(Lib)] public static extern int aexq_weight_replicate(IntPtr ctx, IntPtr w, int batch,
            out IntPtr stack);
        [DllImport(Lib)] public static extern int aexq_weight_alias(IntPtr ctx, IntPtr shared, out IntPtr alias);
        [DllImport(Lib)] public static extern void aexq_weight_release(IntPtr w);
        [DllImport(Lib)] public static extern int aexq_weight_get_info(IntPtr w, out AexqWeightInfo info);

        // ---- execution
        [DllImport(Lib)] public static extern int aexq_plan_check(IntPtr ctx, IntPtr w, ref AexqTensor x,
            ref AexqTensor y, ref AexqLinearArgs args, StringBuilder diag, UIntPtr diagLen);
        [DllImport(Lib)] public static extern int aexq_linear(IntPtr ctx, IntPtr w, ref AexqTensor x,
            ref AexqTensor y, ref AexqLinearArgs args);
        [DllImport(Lib)] public static extern int aexq_linear_group(IntPtr ctx, int count, IntPtr[] w,
            ref AexqTensor x, IntPtr[] y /* AexqTensor* each */, ref AexqLinearArgs args);
        [DllImport(Lib)] public static extern int aexq_lmhead_argmax(IntPtr ctx, IntPtr w, ref AexqTensor x,
            IntPtr logits /* AexqTensor* or 0 */, IntPtr argmax, IntPtr top2Gap);
        [DllImport(Lib)] public static extern int aexq_lmhead_argmax_ex(IntPtr ctx, IntPtr w, ref AexqTensor x,
            IntPtr logits, ref AexqLinearArgs args, IntPtr argmax, IntPtr top2Gap);
        // no counterpart in the reference: for callers that cannot allocate device memory
        [DllImport(Lib)] public static extern int aexq_lmhead_argmax_noalloc(IntPtr ctx, IntPtr w,
            ref AexqTensor x, IntPtr argmax, IntPtr top2Gap);
        [DllImport(Lib)] public static extern int aexq_argmax(IntPtr ctx, ref AexqTensor logits, IntPtr argmax,
            IntPtr top2Gap);
        [DllImport(Lib)] public static extern int aexq_dequant(IntPtr ctx, IntPtr w, IntPtr outF32);

        // ---- decode-step operators around the linears
        [DllImport(Lib)] public static extern int aexq_rmsnorm(IntPtr ctx, ref AexqTensor x, ref AexqTensor y,
            IntPtr gamma, int gammaSize, float eps);
        [DllImport(Lib)] public static extern int aexq_embed_q8(IntPtr ctx, IntPtr table, IntPtr tokens, int m,
            IntPtr outF16);
        [DllImport(Lib)] public static extern int aexq_rope_kv_append(IntPtr ctx, IntPtr q, IntPtr k, IntPtr v,
            IntPtr kCache, IntPtr vCache, int headsQ, int headsKv, int headDim, int capacity, int position,
            IntPtr cosTable, IntPtr sinTable);
        [DllImport(Lib)] public static extern int aexq_attention_decode(IntPtr ctx, IntPtr q, IntPtr kCache,
            IntPtr vCache, int headsQ, int headsKv, int headDim, int capacity, int length, float scale,
            IntPtr outF16);
        [DllImport(Lib)] public static extern int aexq_attention_decode_rope(IntPtr ctx, IntPtr q, IntPtr k,
            IntPtr v, IntPtr kCache, IntPtr vCache, int headsQ, int headsKv, int headDim, int capacity,
            int length, IntPtr cosTable, IntPtr sinTable, float scale, IntPtr outF16);
        [DllImport(Lib)] public static extern int aexq_attention_decode_rope_at(IntPtr ctx, IntPtr q, IntPtr k,
            IntPtr v, IntPtr kCache, IntPtr vCache, int headsQ, int headsKv, int headDim, int capacity,
            IntPtr position /* device int32 */, IntPtr cosTable, IntPtr sinTable, float scale, IntPtr outF16);
        [DllImport(Lib)] public static extern int aexq_decode_advance(IntPtr ctx, IntPtr position, IntPtr token,
            IntPtr argmax, IntPtr tokensOut, int tokensCap);

        // ---- the decoder layers of a decode step in one launch
        [DllImport(Lib)] public static extern int aexq_decoder_create(IntPtr ctx, ref AexqDecoderConfig cfg,
            AexqDecoderLayer[] layers, int count, IntPtr embedding, out IntPtr decoder);
        [DllImport(Lib)] public static extern int aexq_decoder_run(IntPtr decoder, IntPtr token, IntPtr position,
            IntPtr hiddenOutF16);
        [DllImport(Lib)] public static extern int aexq_decoder_error(IntPtr decoder, out int flag);
        [DllImport(Lib)] public static extern int aexq_decoder_info(IntPtr decoder, out int workgroups,
            out int splits, out int splitPositions);
        [DllImport(Lib)] public static extern void aexq_decoder_release(IntPtr decoder);

        /// <summary>The thread's last failure text (never null).</summary>
        public static string LastError()
        {
            return Marshal.PtrToStringAnsi(aexq_last_error()) ?? string.Empty;
        }

        /// <summary>A status as the exception kinds the reference throws for the same
        /// conditions (GL:297-307, IC:421-427, Q8A:282-290).</summary>
        public static void Check(int status, string what)
        {
            if (status == Aexq.Ok)
                return;
            var msg = what + ": " + LastError();
            switch (status)
            {
                case Aexq.ErrInvalidArgument: throw new ArgumentException(msg);
                case Aexq.ErrUnsupported: throw new NotSupportedException(msg);
                case Aexq.ErrShape: throw new InvalidOperationException(msg);
                case Aexq.ErrFormat: throw new System.IO.InvalidDataException(msg);
                case Aexq.ErrOutOfMemory: throw new OutOfMemoryException(msg);
                default: throw new InvalidOperationException(msg + " | status=" + status);
            }
        }
    }
}
