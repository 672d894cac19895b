// The HIP runtime calls the backend makes besides libaexq: device memory for
// the activations it owns, host<->device copies of the per-token int32s, and
// the external-memory / external-semaphore imports through which a blob that a
// Vulkan-backed Unity layer produced becomes a HIP pointer (hip_runtime_api.h;
// the struct offsets are checked against the C compiler by
// tests/test_cpu_host.py).
using System;
using System.Runtime.InteropServices;

namespace Aexis.Hip
{
    [StructLayout(LayoutKind.Explicit, Size = 104)]
    public struct HipExternalMemoryHandleDesc
    {
        [FieldOffset(0)] public int type;          // hipExternalMemoryHandleType
        [FieldOffset(8)] public int fd;            // handle.fd (opaque fd)
        [FieldOffset(8)] public IntPtr win32Handle;
        [FieldOffset(16)] public IntPtr win32Name;
        [FieldOffset(24)] public ulong size;
        [FieldOffset(32)] public uint flags;
    }

    [StructLayout(LayoutKind.Explicit, Size = 88)]
    public struct HipExternalMemoryBufferDesc
    {
        [FieldOffset(0)] public ulong offset;
        [FieldOffset(8)] public ulong size;
        [FieldOffset(16)] public uint flags;
    }

    [StructLayout(LayoutKind.Explicit, Size = 96)]
    public struct HipExternalSemaphoreHandleDesc
    {
        [FieldOffset(0)] public int type;          // hipExternalSemaphoreHandleType
        [FieldOffset(8)] public int fd;
        [FieldOffset(8)] public IntPtr win32Handle;
        [FieldOffset(16)] public IntPtr win32Name;
        [FieldOffset(24)] public uint flags;
    }

    /// <summary>hipExternalSemaphoreSignalParams and ...WaitParams share this size and
    /// the fence value / flags offsets; a binary (opaque fd) semaphore leaves them 0.</summary>
    [StructLayout(LayoutKind.Explicit, Size = 144)]
    public struct HipExternalSemaphoreParams
    {
        [FieldOffset(0)] public ulong fenceValue;
        [FieldOffset(72)] public uint flags;
    }

    public static class AexisHipDevice
    {
        const string Hip = "amdhip64";

        public const int MemcpyHostToDevice = 1;
        public const int MemcpyDeviceToHost = 2;
        public const int ExternalMemoryHandleTypeOpaqueFd = 1;
        public const int ExternalMemoryHandleTypeOpaqueWin32 = 2;
        public const int ExternalSemaphoreHandleTypeOpaqueFd = 1;
        public const int ExternalSemaphoreHandleTypeOpaqueWin32 = 2;

        [DllImport(Hip)] static extern int hipSetDevice(int device);
        [DllImport(Hip)] static extern int hipGetDeviceCount(out int count);
        [DllImport(Hip)] static extern int hipMalloc(out IntPtr ptr, UIntPtr bytes);
        [DllImport(Hip)] static extern int hipFree(IntPtr ptr);
        [DllImport(Hip)] static extern int hipMemsetAsync(IntPtr dst, int value, UIntPtr bytes, IntPtr stream);
        [DllImport(Hip)] static extern int hipMemcpyAsync(IntPtr dst, IntPtr src, UIntPtr bytes, int kind,
            IntPtr stream);
        [DllImport(Hip)] static extern int hipStreamSynchronize(IntPtr stream);
        [DllImport(Hip)] static extern IntPtr hipGetErrorString(int error);
        [DllImport(Hip)] static extern int hipImportExternalMemory(out IntPtr extMem,
            ref HipExternalMemoryHandleDesc desc);
        [DllImport(Hip)] static extern int hipExternalMemoryGetMappedBuffer(out IntPtr devPtr, IntPtr extMem,
            ref HipExternalMemoryBufferDesc desc);
        [DllImport(Hip)] static extern int hipDestroyExternalMemory(IntPtr extMem);
        [DllImport(Hip)] static extern int hipImportExternalSemaphore(out IntPtr extSem,
            ref HipExternalSemaphoreHandleDesc desc);
        [DllImport(Hip)] static extern int hipSignalExternalSemaphoresAsync(IntPtr[] sems,
            HipExternalSemaphoreParams[] prms, uint count, IntPtr stream);
        [DllImport(Hip)] static extern int hipWaitExternalSemaphoresAsync(IntPtr[] sems,
            HipExternalSemaphoreParams[] prms, uint count, IntPtr stream);
        [DllImport(Hip)] static extern int hipDestroyExternalSemaphore(IntPtr extSem);

        /// <summary>The device the backend runs on (AEXIS_HIP_DEVICE, default 0).</summary>
        public static int Ordinal
        {
            get
            {
                var s = Environment.GetEnvironmentVariable("AEXIS_HIP_DEVICE");
                int d;
                return s != null && int.TryParse(s, out d) && d >= 0 ? d : 0;
            }
        }

        static void Check(int err, string what)
        {
            if (err != 0)
                throw new InvalidOperationException(what + " failed: " + Marshal.PtrToStringAnsi(hipGetErrorString(err))
                    + " | status=" + err);
        }

        public static bool Available()
        {
            try
            {
                int n;
                return hipGetDeviceCount(out n) == 0 && n > Ordinal;
            }
            catch (DllNotFoundException)
            {
                return false;
            }
        }

        public static IntPtr Alloc(long bytes)
        {
            Check(hipSetDevice(Ordinal), "hipSetDevice");
            IntPtr p;
            Check(hipMalloc(out p, (UIntPtr)(ulong)Math.Max(bytes, 1)), "hipMalloc(" + bytes + ")");
            return p;
        }

        public static void Free(IntPtr p)
        {
            if (p != IntPtr.Zero)
                hipFree(p);
        }

        public static void Zero(IntPtr p, long bytes, IntPtr stream)
        {
            Check(hipMemsetAsync(p, 0, (UIntPtr)(ulong)bytes, stream), "hipMemsetAsync");
        }

        public static void Upload(IntPtr dst, IntPtr src, long bytes, IntPtr stream)
        {
            Check(hipMemcpyAsync(dst, src, (UIntPtr)(ulong)bytes, MemcpyHostToDevice, stream), "hipMemcpyAsync");
        }

        public static void Download(IntPtr dst, IntPtr src, long bytes, IntPtr stream)
        {
            Check(hipMemcpyAsync(dst, src, (UIntPtr)(ulong)bytes, MemcpyDeviceToHost, stream), "hipMemcpyAsync");
            Check(hipStreamSynchronize(stream), "hipStreamSynchronize");
        }

        /// <summary>Maps `bytes` at `offset` of an exported allocation into HIP. The returned
        /// handle keeps the mapping alive until ReleaseExternal.</summary>
        public static IntPtr ImportExternal(int handleType, int fd, IntPtr win32Handle, long allocationBytes,
                                            long offset, long bytes, out IntPtr devPtr)
        {
            var desc = new HipExternalMemoryHandleDesc
            {
                type = handleType,
                size = (ulong)allocationBytes,
            };
            if (handleType == ExternalMemoryHandleTypeOpaqueFd)
                desc.fd = fd;
            else
                desc.win32Handle = win32Handle;
            IntPtr ext;
            Check(hipImportExternalMemory(out ext, ref desc), "hipImportExternalMemory");
            var buf = new HipExternalMemoryBufferDesc { offset = (ulong)offset, size = (ulong)bytes };
            var err = hipExternalMemoryGetMappedBuffer(out devPtr, ext, ref buf);
            if (err != 0)
            {
                hipDestroyExternalMemory(ext);
                Check(err, "hipExternalMemoryGetMappedBuffer");
            }
            return ext;
        }

        public static void ReleaseExternal(IntPtr ext)
        {
            if (ext != IntPtr.Zero)
                hipDestroyExternalMemory(ext);
        }

        public static IntPtr ImportSemaphore(int handleType, int fd, IntPtr win32Handle)
        {
            var desc = new HipExternalSemaphoreHandleDesc { type = handleType };
            if (handleType == ExternalSemaphoreHandleTypeOpaqueFd)
                desc.fd = fd;
            else
                desc.win32Handle = win32Handle;
            IntPtr sem;
            Check(hipImportExternalSemaphore(out sem, ref desc), "hipImportExternalSemaphore");
            return sem;
        }

        public static void WaitSemaphore(IntPtr sem, IntPtr stream)
        {
            Check(hipWaitExternalSemaphoresAsync(new[] { sem }, new HipExternalSemaphoreParams[1], 1, stream),
                  "hipWaitExternalSemaphoresAsync");
        }

        public static void SignalSemaphore(IntPtr sem, IntPtr stream)
        {
            Check(hipSignalExternalSemaphoresAsync(new[] { sem }, new HipExternalSemaphoreParams[1], 1, stream),
                  "hipSignalExternalSemaphoresAsync");
        }

        public static void ReleaseSemaphore(IntPtr sem)
        {
            if (sem != IntPtr.Zero)
                hipDestroyExternalSemaphore(sem);
        }
    }
}
