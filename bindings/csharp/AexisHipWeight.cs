// A library-owned quantized weight (aexq_weight): the device copy the reference
// makes in NewInt8/Int4WeightOnlyUpload (GS:12834-12996) and keeps in a
// GemmPack's ComputeBuffers (GS:414-455).  An alias shares the tied LM head's
// copy (owns = false, GL:91-111) and is released before its owner.
using System;

namespace Aexis.Hip
{
    public sealed class AexisHipWeight : IDisposable
    {
        public IntPtr Handle { get; private set; }
        public int N { get; }
        public int K { get; }
        public bool Owns { get; }
        readonly AexisHipWeight _owner;   // kept alive while an alias of it exists

        AexisHipWeight(IntPtr handle, bool owns, AexisHipWeight owner)
        {
            Handle = handle;
            Owns = owns;
            _owner = owner;
            AexqWeightInfo info;
            Native.Check(Native.aexq_weight_get_info(handle, out info), "aexq_weight_get_info");
            N = info.n;
            K = info.k;
        }

        public AexqWeightInfo Info()
        {
            AexqWeightInfo info;
            Native.Check(Native.aexq_weight_get_info(Handle, out info), "aexq_weight_get_info");
            return info;
        }

        /// <summary>A direct Q8 record (one fp32 scale per output row; block K, GL:65-67).</summary>
        public static AexisHipWeight Q8(AexisHipContext ctx, AexisQuantizedTensor q, int n, int k, string what)
        {
            IntPtr w;
            Native.Check(Native.aexq_weight_q8(ctx, q.PackedValues, q.Scales, Aexq.DtypeF32, n, k, q.BlockSize,
                                               out w), what);
            return new AexisHipWeight(w, true, null);
        }

        /// <summary>A direct Q4 record (two's-complement nibbles, fp32 scale per block of
        /// BlockSize elements, Q8A:385-413).</summary>
        public static AexisHipWeight Q4(AexisHipContext ctx, AexisQuantizedTensor q, int n, int k, string what)
        {
            IntPtr w;
            Native.Check(Native.aexq_weight_q4(ctx, q.PackedValues, q.Scales, Aexq.DtypeF32, n, k, q.BlockSize,
                                               Aexq.NibbleTwos, out w), what);
            return new AexisHipWeight(w, true, null);
        }

        /// <summary>One AQSGET8 record (header + payload) as AexisGemmLayer.LoadLayer reads it.</summary>
        public static AexisHipWeight FromRecord(AexisHipContext ctx, int bits, byte[] record, int n, int k,
                                                string what, out long consumed)
        {
            IntPtr w;
            UIntPtr used;
            Native.Check(Native.aexq_weight_from_record(ctx, bits, record, (UIntPtr)(ulong)record.Length, n, k,
                                                        out w, out used), what);
            consumed = (long)(ulong)used;
            return new AexisHipWeight(w, true, null);
        }

        /// <summary>Float weights quantized per output row at load time (GS:12838-12964).</summary>
        public static AexisHipWeight FromFloat32(AexisHipContext ctx, int bits, float[] data, int n, int k,
                                                 bool transB, string what)
        {
            IntPtr w;
            var st = bits == 4
                ? Native.aexq_weight_q4_from_f32(ctx, data, n, k, transB ? 1 : 0, out w)
                : Native.aexq_weight_q8_from_f32(ctx, data, n, k, transB ? 1 : 0, out w);
            Native.Check(st, what);
            return new AexisHipWeight(w, true, null);
        }

        /// <summary>A non-owning alias of this weight (the tied embedding / LM head).</summary>
        public AexisHipWeight Alias(AexisHipContext ctx)
        {
            IntPtr w;
            Native.Check(Native.aexq_weight_alias(ctx, Handle, out w), "aexq_weight_alias");
            return new AexisHipWeight(w, false, this);
        }

        public void Dispose()
        {
            if (Handle == IntPtr.Zero)
                return;
            Native.aexq_weight_release(Handle);
            Handle = IntPtr.Zero;
        }
    }
}
