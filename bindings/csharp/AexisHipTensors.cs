// Activations of the HIP-backed layers.  aexq_tensor.data is a HIP device
// pointer; the reference's activations are textures in
// AexisLayerCommandBufferContext.blobs (BL:77-83).  A blob reaches the library
// in one of two ways:
//   1. HIP-resident: a HIP layer produced it (Reserve), so its device buffer
//      and descriptor are here.  The decode path keeps every activation this
//      way, from the token id to the argmax.
//   2. Shared with Unity: a registered IAexisHipExternalBlobSource (a native
//      Vulkan/D3D12 interop plugin) created the blob's storage as exportable
//      memory and hands over its handle; it is imported once with
//      hipImportExternalMemory and mapped as a buffer, and the producer's
//      exported semaphore orders the two APIs.
// Anything else is refused with a NotSupportedException in the reference's
// diagnostic style: there is no texture readback fallback on the inference
// path (the strict plan, TEP:389-407).
using System;
using System.Collections.Generic;
using Aexis.Execution;

namespace Aexis.Hip
{
    /// <summary>A blob's storage exported by the graphics API (Pack4 texel rows,
    /// LinearMat rows or a linear buffer).</summary>
    public struct AexisHipExternalBlob
    {
        public int handleType;          // AexisHipDevice.ExternalMemoryHandleType*
        public int fd;                  // opaque fd (Vulkan)
        public IntPtr win32Handle;      // NT handle (D3D12 / Vulkan on Windows)
        public long allocationBytes;    // size of the exported allocation
        public long offset;             // the blob's first byte inside it
        public long rowPitchBytes;      // bytes between storage rows as the driver laid them out
        public int layout;              // Aexq.Layout*
        public int dtype;               // Aexq.Dtype* (RGBA16F -> F16, RGBA32F -> F32)
        public int semaphoreHandleType; // 0: no semaphore (the producer finished on the host)
        public int semaphoreFd;
        public IntPtr semaphoreWin32Handle;
    }

    /// <summary>Implemented by the graphics-interop plugin that owns exportable textures.</summary>
    public interface IAexisHipExternalBlobSource
    {
        /// <summary>The exported storage of an input blob produced by a Unity layer.</summary>
        bool TryExport(AexisLayerCommandBufferContext context, string blob, out AexisHipExternalBlob exported);

        /// <summary>Creates an exportable texture for an output blob that Unity layers will
        /// read, publishes it in context.blobs / context.shapes, and returns its storage.</summary>
        bool TryCreateShared(AexisLayerCommandBufferContext context, string blob,
                             AexisGraphSession.BufferShape logical, AexisGraphSession.BufferShape storage,
                             int dtype, out AexisHipExternalBlob exported);
    }

    public sealed class AexisHipTensors : IDisposable
    {
        sealed class Blob
        {
            public IntPtr data;
            public long bytes;
            public AexqTensor desc;
            public bool owned;      // hipMalloc'ed here
            public IntPtr extMem;   // imported external memory (0: none)
            public int extFd;
            public IntPtr semaphore;
        }

        /// <summary>The interop plugin, when one is loaded (null: HIP-resident blobs only).</summary>
        public static IAexisHipExternalBlobSource ExternalSource { get; set; }

        readonly AexisHipContext _ctx;
        readonly Dictionary<string, Blob> _blobs = new Dictionary<string, Blob>(StringComparer.Ordinal);

        internal AexisHipTensors(AexisHipContext ctx)
        {
            _ctx = ctx;
        }

        // ---- storage rules (GS:10836-10852, GL:515-525, GL:1003-1043)

        public static AexisGraphSession.BufferShape Logical(int rows, int width)
        {
            return new AexisGraphSession.BufferShape(2, Math.Max(1, width), Math.Max(1, rows), 1, 1);
        }

        public static AexisGraphSession.BufferShape Storage(int layout, int rows, int width, int headDim = 0)
        {
            rows = Math.Max(1, rows);
            var packs = (Math.Max(1, width) + 3) / 4;
            switch (layout)
            {
                case Aexq.LayoutLinear:
                    return new AexisGraphSession.BufferShape(2, width, rows, 1, 1);
                case Aexq.LayoutPack4Linear:
                    return new AexisGraphSession.BufferShape(3, packs, rows, 1, 4);
                case Aexq.LayoutPack4Tiled:
                {
                    var tileW = Math.Min(packs, Math.Max(1, Math.Min(Aexq.TileWidthLimit, MaxTextureSize)));
                    var tileRows = (packs + tileW - 1) / tileW;
                    return new AexisGraphSession.BufferShape(3, tileW, rows * tileRows, 1, 4);
                }
                case Aexq.LayoutHeadPacked:
                    if (headDim <= 0 || width % headDim != 0)
                        throw new InvalidOperationException("width " + width + " is not heads x head_dim " + headDim);
                    return new AexisGraphSession.BufferShape(3, headDim, rows, 1, width / headDim);
                default:
                    throw new NotSupportedException("layout " + layout + " has no storage rule");
            }
        }

        /// <summary>Elements of a [rows][width] tensor in the layout's storage.</summary>
        public static long Elements(int layout, int rows, int width, int headDim = 0)
        {
            var s = Storage(layout, rows, width, headDim);
            if (layout == Aexq.LayoutHeadPacked)
                return (long)((s.c + 3) / 4) * s.h * s.w * 4;
            return (long)s.w * s.h * (layout == Aexq.LayoutLinear ? 1 : 4);
        }

        /// <summary>GL:515-525: tiled when ceil(n/4) exceeds the texture limit, else Pack4 linear
        /// when n % 4 == 0, else LinearMat.</summary>
        public static int OutputLayoutFor(int n)
        {
            if ((n + 3) / 4 > MaxTextureSize)
                return Aexq.LayoutPack4Tiled;
            return n % 4 == 0 ? Aexq.LayoutPack4Linear : Aexq.LayoutLinear;
        }

        static int MaxTextureSize
        {
            get { return Math.Max(1, UnityEngine.SystemInfo.maxTextureSize); }
        }

        static AexqShape ToAexq(AexisGraphSession.BufferShape s)
        {
            return new AexqShape(s.dims, s.w, s.h, s.d, s.c);
        }

        static string Diag(string what, string blob, string detail)
        {
            return what + " | blob=" + blob + " | " + detail + " | rejectedFallback=texture-readback";
        }

        // ---- the two entry points the layer uses

        /// <summary>The blob as the library reads it, with its logical shape from
        /// context.shapes (BL:77-83).</summary>
        public static AexqTensor Describe(AexisGraphSession owner, AexisLayerCommandBufferContext context,
                                          string blob)
        {
            return AexisHipContext.For(owner).Tensors.Import(context, blob);
        }

        /// <summary>A device output blob of rows x width in `layout`; its logical shape is
        /// published in context.shapes for the layers that follow.</summary>
        public static AexqTensor Allocate(AexisGraphSession owner, AexisLayerCommandBufferContext context,
                                          string blob, int rows, int width, int layout, int dtype = Aexq.DtypeF16,
                                          int headDim = 0)
        {
            return AexisHipContext.For(owner).Tensors.Reserve(context, blob, rows, width, layout, dtype, headDim);
        }

        public AexqTensor Import(AexisLayerCommandBufferContext context, string blob)
        {
            if (context == null)
                throw new ArgumentNullException(nameof(context));
            Blob b;
            if (_blobs.TryGetValue(blob, out b))
            {
                if (b.semaphore != IntPtr.Zero)
                    AexisHipDevice.WaitSemaphore(b.semaphore, _ctx.Stream);
                return b.desc;
            }
            AexisGraphSession.BufferShape logical;
            if (context.shapes == null || !context.shapes.TryGetValue(blob, out logical))
                throw new InvalidOperationException(Diag("input blob has no logical shape", blob, "shapes=missing"));
            if (logical.dims != 2)
                throw new NotSupportedException(Diag("the quantized Gemm reads 2-D inputs", blob,
                                                     "dims=" + logical.dims));
            AexisHipExternalBlob ext;
            var src = ExternalSource;
            if (src == null || !src.TryExport(context, blob, out ext))
                throw new NotSupportedException(Diag(
                    "input blob is a Unity texture that is not exportable to HIP", blob,
                    "interop=" + (src == null ? "none" : "declined")));
            return Map(blob, logical.h, logical.w, ext, 0);
        }

        public AexqTensor Reserve(AexisLayerCommandBufferContext context, string blob, int rows, int width,
                                  int layout, int dtype = Aexq.DtypeF16, int headDim = 0)
        {
            if (context == null)
                throw new ArgumentNullException(nameof(context));
            var logical = Logical(rows, width);
            var storage = Storage(layout, rows, width, headDim);
            var bytes = Elements(layout, rows, width, headDim) * (dtype == Aexq.DtypeF32 ? 4 : 2);
            Blob b;
            if (_blobs.TryGetValue(blob, out b) && b.bytes == bytes && b.desc.layout == layout
                && b.desc.dtype == dtype && b.desc.logical.w == logical.w && b.desc.logical.h == logical.h)
            {
                context.shapes[blob] = logical;
                return b.desc;
            }
            if (b != null)
                Drop(blob, b);
            AexisHipExternalBlob ext;
            var src = ExternalSource;
            if (src != null && src.TryCreateShared(context, blob, logical, storage, dtype, out ext))
            {
                context.shapes[blob] = logical;
                return Map(blob, rows, width, ext, headDim);
            }
            b = new Blob { data = AexisHipDevice.Alloc(bytes), bytes = bytes, owned = true };
            AexisHipDevice.Zero(b.data, bytes, _ctx.Stream);   // Pack4 tail lanes read as zero
            b.desc = new AexqTensor
            {
                logical = ToAexq(logical),
                storage = ToAexq(storage),
                layout = layout,
                dtype = dtype,
                data = b.data,
                batch = 1,
                batchStride = 0,
            };
            _blobs[blob] = b;
            context.shapes[blob] = logical;
            return b.desc;
        }

        AexqTensor Map(string blob, int rows, int width, AexisHipExternalBlob ext, int headDim)
        {
            var storage = Storage(ext.layout, rows, width, headDim);
            var elementBytes = ext.dtype == Aexq.DtypeF32 ? 4 : 2;
            var bytes = Elements(ext.layout, rows, width, headDim) * elementBytes;
            var denseRow = ext.layout == Aexq.LayoutLinear ? (long)width * elementBytes
                : ext.layout == Aexq.LayoutHeadPacked ? (long)headDim * 4 * elementBytes
                : (long)storage.w * 4 * elementBytes;
            if (rows > 1 && ext.rowPitchBytes != 0 && ext.rowPitchBytes != denseRow)
                throw new NotSupportedException(Diag("exported rows are padded", blob,
                    "rowPitch=" + ext.rowPitchBytes + " | denseRow=" + denseRow));
            if (ext.offset + bytes > ext.allocationBytes)
                throw new InvalidOperationException(Diag("exported allocation is smaller than the blob", blob,
                    "allocation=" + ext.allocationBytes + " | need=" + (ext.offset + bytes)));
            IntPtr dev;
            var mem = AexisHipDevice.ImportExternal(ext.handleType, ext.fd, ext.win32Handle, ext.allocationBytes,
                                                    ext.offset, bytes, out dev);
            var b = new Blob { data = dev, bytes = bytes, extMem = mem, extFd = ext.fd };
            if (ext.semaphoreHandleType != 0)
                b.semaphore = AexisHipDevice.ImportSemaphore(ext.semaphoreHandleType, ext.semaphoreFd,
                                                             ext.semaphoreWin32Handle);
            b.desc = new AexqTensor
            {
                logical = ToAexq(Logical(rows, width)),
                storage = ToAexq(storage),
                layout = ext.layout,
                dtype = ext.dtype,
                data = dev,
                batch = 1,
                batchStride = 0,
            };
            _blobs[blob] = b;
            if (b.semaphore != IntPtr.Zero)
                AexisHipDevice.WaitSemaphore(b.semaphore, _ctx.Stream);
            return b.desc;
        }

        /// <summary>Hands an output that Unity layers read back to the graphics queue.</summary>
        public void Publish(string blob)
        {
            Blob b;
            if (_blobs.TryGetValue(blob, out b) && b.semaphore != IntPtr.Zero)
                AexisHipDevice.SignalSemaphore(b.semaphore, _ctx.Stream);
        }

        public bool TryGet(string blob, out AexqTensor desc)
        {
            Blob b;
            if (_blobs.TryGetValue(blob, out b))
            {
                desc = b.desc;
                return true;
            }
            desc = default(AexqTensor);
            return false;
        }

        void Drop(string blob, Blob b)
        {
            _ctx.Synchronize();
            if (b.owned)
                AexisHipDevice.Free(b.data);
            AexisHipDevice.ReleaseExternal(b.extMem);
            AexisHipDevice.ReleaseSemaphore(b.semaphore);
            _blobs.Remove(blob);
        }

        public void Dispose()
        {
            foreach (var b in _blobs.Values)
            {
                if (b.owned)
                    AexisHipDevice.Free(b.data);
                AexisHipDevice.ReleaseExternal(b.extMem);
                AexisHipDevice.ReleaseSemaphore(b.semaphore);
            }
            _blobs.Clear();
        }
    }
}
