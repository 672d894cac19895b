// One libaexq context per graph session.  The reference keeps one AexisOps
// (dispatch state) per session (OPS:706-760); the backend keeps one aexq_ctx
// (device, HIP stream, grown scratch) per AexisGraphSession the same way,
// created on first use and destroyed with the session or on Dispose.
using System;
using System.Runtime.CompilerServices;
using Aexis.Execution;

namespace Aexis.Hip
{
    public sealed class AexisHipContext : IDisposable
    {
        static readonly ConditionalWeakTable<AexisGraphSession, AexisHipContext> s_bySession =
            new ConditionalWeakTable<AexisGraphSession, AexisHipContext>();

        public IntPtr Handle { get; private set; }
        public int Device { get; }
        public IntPtr Stream { get; private set; }
        public readonly AexisHipTensors Tensors;

        public AexisHipContext(int device, IntPtr hipStream)
        {
            var abi = Native.aexq_abi_version();
            if (abi != Aexq.AbiVersion)
                throw new NotSupportedException("libaexq ABI " + abi + " | expected=" + Aexq.AbiVersion
                                                + " | rejectedFallback=none");
            IntPtr h;
            Native.Check(Native.aexq_create(device, hipStream, out h), "aexq_create");
            Handle = h;
            Device = device;
            Stream = hipStream;
            Tensors = new AexisHipTensors(this);
        }

        /// <summary>The session's context (created on the backend's device and the null
        /// stream on first use).</summary>
        public static AexisHipContext For(AexisGraphSession owner)
        {
            if (owner == null)
                throw new ArgumentNullException(nameof(owner));
            return s_bySession.GetValue(owner, s => new AexisHipContext(AexisHipDevice.Ordinal, IntPtr.Zero));
        }

        /// <summary>Drops the session's context (its tensors, then the library context).</summary>
        public static void Release(AexisGraphSession owner)
        {
            AexisHipContext c;
            if (owner != null && s_bySession.TryGetValue(owner, out c))
            {
                s_bySession.Remove(owner);
                c.Dispose();
            }
        }

        public void SetStream(IntPtr hipStream)
        {
            Native.Check(Native.aexq_set_stream(Handle, hipStream), "aexq_set_stream");
            Stream = hipStream;
        }

        public void Synchronize()
        {
            Native.Check(Native.aexq_synchronize(Handle), "aexq_synchronize");
        }

        public static implicit operator IntPtr(AexisHipContext c)
        {
            return c.Handle;
        }

        public void Dispose()
        {
            if (Handle == IntPtr.Zero)
                return;
            Native.aexq_synchronize(Handle);
            Tensors.Dispose();
            Native.aexq_destroy(Handle);
            Handle = IntPtr.Zero;
        }
    }
}
