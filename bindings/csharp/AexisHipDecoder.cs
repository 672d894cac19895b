// The decode step of Qwen35DecoderSession (DEC:463-809) on libaexq: the fused
// decoder layers (aexq_decoder_run: embedding gather and every layer in one
// launch), the LM head with the final RMSNorm and the greedy argmax fused
// (aexq_lmhead_argmax_ex), and Generate's feedback of the token
// (aexq_decode_advance, DEC:1160-1237).  The token and the position stay in
// device memory, so the three calls replay token after token; the host reads
// one int32 per generated position when it wants the text.  A model the fused
// kernel does not take is refused at creation with
// "rejectedFallback=per-operator step"; the caller then binds the
// per-operator calls (INTEGRATION.md, decode-step operators).
using System;
using System.Runtime.InteropServices;

namespace Aexis.Hip
{
    public sealed class AexisHipDecoderLayer
    {
        public AexisHipWeight qProj, kProj, vProj, oProj, gateProj, upProj, downProj;
        public float[] attnNorm, mlpNorm;   // RMSNorm gammas [hidden]
    }

    public sealed class AexisHipDecoder : IDisposable
    {
        readonly AexisHipContext _ctx;
        readonly AexisHipWeight _lmHead;
        readonly AexisHipWeight _embed;      // alias of the LM head (the tied table)
        readonly AexisHipDecoderLayer[] _layers;
        readonly int _hidden, _capacity;
        readonly float _eps;
        IntPtr _decoder;
        IntPtr _norms, _caches, _rope, _finalNorm, _state, _history;
        IntPtr _hiddenState;
        AexqTensor _hiddenDesc;

        // device int32 words of _state
        const int TokenWord = 0, PositionWord = 1, ArgmaxWord = 2;

        public int Capacity
        {
            get { return _capacity; }
        }

        /// <summary>Uploads the norms, zeroes fp16 K/V caches of `capacity` positions, builds the
        /// RoPE rows of every position (DEC:1660-1675) and creates the fused decoder.</summary>
        public AexisHipDecoder(AexisHipContext ctx, AexisHipDecoderLayer[] layers, AexisHipWeight lmHead,
                               float[] finalNorm, int headsQ, int headsKv, int headDim, int capacity,
                               float rmsEps, float ropeTheta)
        {
            if (layers == null || layers.Length == 0)
                throw new ArgumentException("no layers");
            _ctx = ctx;
            _layers = layers;
            _lmHead = lmHead;
            _hidden = lmHead.K;
            _capacity = capacity;
            _eps = rmsEps;
            _embed = lmHead.Alias(ctx);
            var hd = _hidden;
            var kvBytes = (long)headsKv * capacity * headDim * 2;
            _norms = AexisHipDevice.Alloc((long)layers.Length * 2 * hd * 4);
            _caches = AexisHipDevice.Alloc((long)layers.Length * 2 * kvBytes);
            AexisHipDevice.Zero(_caches, (long)layers.Length * 2 * kvBytes, ctx.Stream);
            var half = headDim / 2;
            _rope = AexisHipDevice.Alloc(2L * capacity * half * 4);
            _finalNorm = AexisHipDevice.Alloc((long)hd * 4);
            _state = AexisHipDevice.Alloc(256);
            AexisHipDevice.Zero(_state, 256, ctx.Stream);
            _history = AexisHipDevice.Alloc((long)capacity * 4);
            _hiddenState = AexisHipDevice.Alloc((long)hd * 2);

            var table = new AexqDecoderLayer[layers.Length];
            for (var l = 0; l < layers.Length; ++l)
            {
                var L = layers[l];
                var gA = Offset(_norms, (2L * l) * hd * 4);
                var gM = Offset(_norms, (2L * l + 1) * hd * 4);
                Put(gA, L.attnNorm);
                Put(gM, L.mlpNorm);
                table[l] = new AexqDecoderLayer
                {
                    qProj = L.qProj.Handle, kProj = L.kProj.Handle, vProj = L.vProj.Handle,
                    oProj = L.oProj.Handle, gateProj = L.gateProj.Handle, upProj = L.upProj.Handle,
                    downProj = L.downProj.Handle,
                    attnNorm = gA, mlpNorm = gM,
                    kCache = Offset(_caches, (2L * l) * kvBytes),
                    vCache = Offset(_caches, (2L * l + 1) * kvBytes),
                };
            }
            float[] cos, sin;
            RopeTables(capacity, headDim, ropeTheta, out cos, out sin);
            Put(_rope, cos);
            Put(Offset(_rope, (long)capacity * half * 4), sin);
            Put(_finalNorm, finalNorm);
            ctx.Synchronize();
            var cfg = new AexqDecoderConfig
            {
                headsQ = headsQ, headsKv = headsKv, headDim = headDim, capacity = capacity,
                rmsEps = rmsEps, attnScale = (float)(1.0 / Math.Sqrt(headDim)),
                ropeCos = _rope, ropeSin = Offset(_rope, (long)capacity * half * 4), workgroups = 0,
            };
            Native.Check(Native.aexq_decoder_create(ctx, ref cfg, table, table.Length, _embed.Handle,
                                                    out _decoder), "aexq_decoder_create");
            _hiddenDesc = new AexqTensor
            {
                logical = new AexqShape(2, hd, 1, 1, 1),
                storage = new AexqShape(3, (hd + 3) / 4, 1, 1, 4),
                layout = Aexq.LayoutPack4Linear,
                dtype = Aexq.DtypeF16,
                data = _hiddenState,
                batch = 1,
            };
        }

        static IntPtr Offset(IntPtr p, long bytes)
        {
            return new IntPtr(p.ToInt64() + bytes);
        }

        void Put(IntPtr dst, float[] src)
        {
            var pin = GCHandle.Alloc(src, GCHandleType.Pinned);
            try
            {
                AexisHipDevice.Upload(dst, pin.AddrOfPinnedObject(), (long)src.Length * 4, _ctx.Stream);
                _ctx.Synchronize();
            }
            finally
            {
                pin.Free();
            }
        }

        /// <summary>CreateRopeTextures' rows for every position (DEC:1660-1675), in its float32
        /// steps: row p holds cos / sin of p * (1 / theta^(2j / d)).</summary>
        public static void RopeTables(int capacity, int headDim, float theta, out float[] cos, out float[] sin)
        {
            var half = headDim / 2;
            cos = new float[capacity * half];
            sin = new float[capacity * half];
            var step = 2f / (half * 2f);
            for (var j = 0; j < half; ++j)
            {
                var e = j * step;
                var inverse = 1f / (float)Math.Pow(theta, e);
                for (var p = 0; p < capacity; ++p)
                {
                    var angle = p * inverse;
                    cos[p * half + j] = (float)Math.Cos(angle);
                    sin[p * half + j] = (float)Math.Sin(angle);
                }
            }
        }

        /// <summary>Sets the next input token and its position (a prompt's last token).</summary>
        public void Start(int token, int position)
        {
            if (position < 0 || position >= _capacity)
                throw new ArgumentOutOfRangeException(nameof(position));
            var words = new[] { token, position };
            var pin = GCHandle.Alloc(words, GCHandleType.Pinned);
            try
            {
                AexisHipDevice.Upload(_state, pin.AddrOfPinnedObject(), 8, _ctx.Stream);
                _ctx.Synchronize();
            }
            finally
            {
                pin.Free();
            }
        }

        /// <summary>One greedy token: layers, final norm + LM head + argmax, then the token and
        /// position advance on the device.  Asynchronous; allocates nothing, so it can be
        /// captured into a HIP graph.</summary>
        public void Step()
        {
            Native.Check(Native.aexq_decoder_run(_decoder, Offset(_state, TokenWord * 4),
                                                 Offset(_state, PositionWord * 4), _hiddenState), "aexq_decoder_run");
            var args = AexqLinearArgs.Default();
            args.rmsGamma = _finalNorm;
            args.rmsGammaSize = _hidden;
            args.rmsEps = _eps;
            args.flags = Aexq.EpiRmsNormIn;
            Native.Check(Native.aexq_lmhead_argmax_ex(_ctx, _lmHead.Handle, ref _hiddenDesc, IntPtr.Zero, ref args,
                                                      Offset(_state, ArgmaxWord * 4), IntPtr.Zero), "lm head");
            Native.Check(Native.aexq_decode_advance(_ctx, Offset(_state, PositionWord * 4),
                                                    Offset(_state, TokenWord * 4), Offset(_state, ArgmaxWord * 4),
                                                    _history, _capacity), "aexq_decode_advance");
        }

        /// <summary>Greedy decoding of `count` tokens after Start (Generate, DEC:1160-1237).</summary>
        public int[] Generate(int startToken, int position, int count)
        {
            if (count < 0 || position + count > _capacity)
                throw new ArgumentOutOfRangeException(nameof(count));
            Start(startToken, position);
            for (var i = 0; i < count; ++i)
                Step();
            int flag;
            Native.Check(Native.aexq_decoder_error(_decoder, out flag), "aexq_decoder_error");
            if (flag != 0)
                throw new InvalidOperationException("aexq_decoder_run gave up a bounded wait: the tokens are invalid");
            var all = new int[_capacity];
            var pin = GCHandle.Alloc(all, GCHandleType.Pinned);
            try
            {
                AexisHipDevice.Download(pin.AddrOfPinnedObject(), _history, (long)_capacity * 4, _ctx.Stream);
            }
            finally
            {
                pin.Free();
            }
            var tokens = new int[count];
            Array.Copy(all, position, tokens, 0, count);
            return tokens;
        }

        public void Dispose()
        {
            if (_decoder != IntPtr.Zero)
            {
                _ctx.Synchronize();
                Native.aexq_decoder_release(_decoder);
                _decoder = IntPtr.Zero;
            }
            _embed.Dispose();
            foreach (var p in new[] { _norms, _caches, _rope, _finalNorm, _state, _history, _hiddenState })
                AexisHipDevice.Free(p);
            _norms = _caches = _rope = _finalNorm = _state = _history = _hiddenState = IntPtr.Zero;
        }
    }
}
