// AexisHipGemmLayer: the quantized Gemm on libaexq, a drop-in for
// AexisGemmLayer (Packages/com.aexis/Runtime/Execution/Layers/AexisGemmLayer.cs,
// GL below) on the transB, constant-B path that Qwen3.5 decode runs.  Load
// time follows GL:15-162 (param ids 0..10, the constantA refusal, the shared
// tied LM head, direct Q4 / Q8 records, per-row re-quantization of anything
// else); execution replaces TryExecuteCommandBufferTexturePath (GL:327-469)
// with one aexq_linear call on the session's HIP stream.  Whatever the library
// has no kernel for fails with the library's diagnostic; nothing falls back.
using System;
using System.Collections.Generic;
using System.Runtime.InteropServices;
using System.Text;
using Aexis.Execution;

namespace Aexis.Hip
{
    /// <summary>Reads the next AQSGET8 record's bytes (24-byte header + payload,
    /// NcnnQ8Archive.cs:236-339) without consuming them, and skips what the library
    /// consumed.  Implemented by the archive-backed AexisWeightReader of the fork that
    /// ships this backend; readers without an archive take the typed path (WR:16-21).</summary>
    public interface IAexisArchiveRecordSource
    {
        byte[] PeekRecordBytes();
        void Skip(long bytes);
    }

    public sealed class AexisHipGemmLayer : AexisBaseLayer
    {
        public const string KernelId = "aexq.gemm";

        // Shared weights by session and element count: the tied embedding / LM head the
        // decode driver uploads once (GL:91-111, EMB:95-120).  A Gemm whose weight has
        // the shared element count aliases it instead of reading its own copy.
        static readonly Dictionary<AexisGraphSession, AexisHipWeight> s_shared =
            new Dictionary<AexisGraphSession, AexisHipWeight>();
        static readonly object s_gate = new object();

        // Gemm layers whose output feeds Reshape -> Permute(2) -> SDPA, by layer name, with
        // the head size: their output is stored head-packed (GL:1003-1043).  The decode
        // driver that owns the model's layout registers them.
        static readonly Dictionary<string, int> s_headPacked = new Dictionary<string, int>(StringComparer.Ordinal);

        AexisHipWeight _weight;
        AexqLinearArgs _args;
        IntPtr _bias;
        int _n, _k;
        int _headDim;           // > 0: q/k/v projection writing the head-packed layout
        string _name;

        public AexisHipGemmLayer() : base(AexisLayerTypes.Gemm, supportsBufferPath: false,
                                          supportsCommandBufferPath: true) { }

        /// <summary>The tied LM head of `owner`, shared by the embedding gather and the
        /// LM-head Gemm (owns = false on the Gemm side).</summary>
        public static void SetSharedWeight(AexisGraphSession owner, AexisHipWeight weight)
        {
            lock (s_gate)
                s_shared[owner] = weight;
        }

        public static void ReleaseSession(AexisGraphSession owner)
        {
            lock (s_gate)
                s_shared.Remove(owner);
        }

        public static void SetHeadPackedOutput(string layerName, int headDim)
        {
            lock (s_gate)
                s_headPacked[layerName] = headDim;
        }

        public AexisHipWeight Weight
        {
            get { return _weight; }
        }

        static string Diag(AexisGraphModel.Layer layer, string reason)
        {
            return reason + " | layer=" + (layer.name ?? string.Empty) + " | type=Gemm"
                   + " | rejectedFallback=AexisGemmLayer";
        }

        public override AexisGraphSession.LayerLoadMetrics LoadLayer(AexisGraphSession owner,
                                                                     AexisGraphModel.Layer layer,
                                                                     AexisWeightReader br)
        {
            if (owner == null)
                throw new ArgumentNullException(nameof(owner));
            if (layer == null)
                throw new ArgumentNullException(nameof(layer));
            _name = layer.name;
            // ncnn Gemm params (GL:23-34)
            var alpha = layer.GetFloat(0, 1f);
            var beta = layer.GetFloat(1, 1f);
            var transA = layer.GetInt(2, 0) != 0;
            var transB = layer.GetInt(3, 0) != 0;
            var constantA = layer.GetInt(4, 0) != 0;
            var constantB = layer.GetInt(5, 0) != 0;
            var constantC = layer.GetInt(6, 0) != 0;
            var constantM = layer.GetInt(7, 0);
            _n = layer.GetInt(8, 0);
            _k = layer.GetInt(9, 0);
            var broadcastC = layer.GetInt(10, 0);
            if (constantA)
                throw new InvalidOperationException("Gemm constantA is not supported in AexisGraphSession: " + layer.name);
            if (!constantB || transA)
                throw new NotSupportedException(Diag(layer, "the HIP Gemm takes a constant B and a plain A"));
            if (_n <= 0 || _k <= 0)
                throw new InvalidOperationException(Diag(layer, "constantN=" + _n + " constantK=" + _k));

            var ctx = AexisHipContext.For(owner);
            var int4 = owner.UsesInt4WeightOnlyForLayer(layer);
            var int8 = owner.UsesInt8WeightOnlyForLayer(layer);
            if (!int4 && !int8)
                throw new NotSupportedException(Diag(layer, "the HIP Gemm runs quantized weight-only layers"));
            var bw = transB ? _k : _n;
            var bh = transB ? _n : _k;
            var count = (long)_n * _k;

            AexisHipWeight shared = null;
            lock (s_gate)
                s_shared.TryGetValue(owner, out shared);
            if (shared != null && owner.SharedTokenEmbeddingElementCount == count && shared.N == _n && shared.K == _k)
            {
                br.SkipTensor(bw, bh, 0, 0, 0);                    // GL:56-57
                _weight = shared.Alias(ctx);
            }
            else
            {
                var records = br as IAexisArchiveRecordSource;
                AexisQuantizedTensor direct;
                if (records != null && transB)
                {
                    // the record as stored: the library repacks a Q4 record (int4 layer) or a
                    // Q8 record with block K (int8 layer) on the device and quantizes any other
                    // record per output row, the three outcomes of GL:60-141
                    var rec = records.PeekRecordBytes();
                    _weight = AexisHipWeight.FromRecord(ctx, int4 ? 4 : 8, rec, _n, _k, layer.name, out var used);
                    records.Skip(used);
                }
                else if (int4 && transB && br.TryReadInt4QuantizedTensor((int)count, _k, out direct))
                    _weight = AexisHipWeight.Q4(ctx, direct, _n, _k, layer.name);          // WR:21, GS:12966-12996
                else if (int8 && transB && br.TryReadQuantizedTensor((int)count, _k, out direct))
                    _weight = AexisHipWeight.Q8(ctx, direct, _n, _k, layer.name);          // WR:16, GS:12887-12907
                else
                {
                    // GS:12838-12885 / 12912-12964: float weights quantized per output channel
                    var f = br.ReadTensorAsFloat32(bw, bh, 0, 0, 0);
                    _weight = AexisHipWeight.FromFloat32(ctx, int4 ? 4 : 8, f, _n, _k, transB, layer.name);
                }
            }

            _args = AexqLinearArgs.Default();
            _args.alpha = alpha;
            _args.beta = beta;
            if (constantC && broadcastC != -1)
            {
                int cw, ch;
                switch (broadcastC)                               // GL:70-82
                {
                    case 0: cw = 1; ch = 0; break;
                    case 1: cw = constantM; ch = 0; break;
                    case 3: cw = _n; ch = constantM; break;
                    case 4: cw = _n; ch = 1; break;
                    default:
                        throw new NotSupportedException(Diag(layer, "broadcast_type_C=" + broadcastC));
                }
                var c = br.ReadTensorAsFloat32(cw, ch, 0, 0, 0);
                _bias = AexisHipDevice.Alloc((long)c.Length * 4);
                var pin = GCHandle.Alloc(c, GCHandleType.Pinned);
                try
                {
                    AexisHipDevice.Upload(_bias, pin.AddrOfPinnedObject(), (long)c.Length * 4, ctx.Stream);
                    ctx.Synchronize();
                }
                finally
                {
                    pin.Free();
                }
                _args.c = _bias;
                _args.broadcastC = broadcastC;
            }
            lock (s_gate)
                s_headPacked.TryGetValue(layer.name ?? string.Empty, out _headDim);
            return default(AexisGraphSession.LayerLoadMetrics);
        }

        public override void ExecuteRenderTexturePath(AexisGraphSession owner, AexisGraphModel.Layer layer,
                                                      AexisLayerBufferContext context)
        {
            throw new NotSupportedException(Diag(layer, "the HIP Gemm runs on the CommandBuffer path"));
        }

        public override void ExecuteCommandBuffer(AexisGraphSession owner, AexisGraphModel.Layer layer,
                                                  AexisLayerCommandBufferContext context)
        {
            if (owner == null)
                throw new ArgumentNullException(nameof(owner));
            if (layer == null)
                throw new ArgumentNullException(nameof(layer));
            if (context == null)
                throw new ArgumentNullException(nameof(context));
            if (_weight == null)
                throw new InvalidOperationException(Diag(layer, "LoadLayer has not run"));
            var ctx = AexisHipContext.For(owner);
            var x = AexisHipTensors.Describe(owner, context, layer.bottomNames[0]);
            var m = x.logical.h;
            if (x.logical.w != _k)
                throw new InvalidOperationException(Diag(layer, "input width " + x.logical.w + " != K " + _k));
            var layout = _headDim > 0 ? Aexq.LayoutHeadPacked : AexisHipTensors.OutputLayoutFor(_n);
            var y = AexisHipTensors.Allocate(owner, context, layer.topNames[0], m, _n, layout, Aexq.DtypeF16,
                                             _headDim);
            Native.Check(Native.aexq_linear(ctx, _weight.Handle, ref x, ref y, ref _args), layer.name);
            ctx.Tensors.Publish(layer.topNames[0]);
        }

        /// <summary>Strict preflight (TEP:252-261, 389-407): the library's verdict for this layer
        /// at `rows` activation rows, or null when a kernel exists.</summary>
        public string PlanCheck(AexisGraphSession owner, int rows)
        {
            if (_weight == null)
                return "LoadLayer has not run | layer=" + _name;
            var ctx = AexisHipContext.For(owner);
            var x = new AexqTensor
            {
                logical = new AexqShape(2, _k, rows, 1, 1),
                storage = new AexqShape(3, (_k + 3) / 4, rows, 1, 4),
                layout = Aexq.LayoutPack4Linear,
                dtype = Aexq.DtypeF16,
                batch = 1,
            };
            var layout = _headDim > 0 ? Aexq.LayoutHeadPacked : AexisHipTensors.OutputLayoutFor(_n);
            var s = AexisHipTensors.Storage(layout, rows, _n, _headDim);
            var y = new AexqTensor
            {
                logical = new AexqShape(2, _n, rows, 1, 1),
                storage = new AexqShape(s.dims, s.w, s.h, s.d, s.c),
                layout = layout,
                dtype = Aexq.DtypeF16,
                batch = 1,
            };
            var diag = new StringBuilder(1024);
            var st = Native.aexq_plan_check(ctx, _weight.Handle, ref x, ref y, ref _args, diag,
                                            (UIntPtr)diag.Capacity);
            return st == Aexq.Ok ? null : diag.ToString();
        }

        /// <summary>Registers the layer for `Gemm` when the HIP backend is active
        /// (AexisCustomLayerRegistry.Register, AexisCustomLayerRegistry.cs:160).</summary>
        public static void Register()
        {
            AexisCustomLayerRegistry.Register(new AexisCustomLayerDefinition
            {
                typeName = "Gemm",
                kernelId = KernelId,
                schema = new AexisCustomLayerSchema { minimumInputs = 1, maximumInputs = 1, maximumOutputs = 1 },
                createLayer = () => new AexisHipGemmLayer(),
            }, replaceExisting: true);
        }
    }
}
