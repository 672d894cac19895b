// Switching a session's quantized Gemm layers to libaexq, and the strict
// preflight over them.  Register() swaps the Gemm factory entry for
// AexisHipGemmLayer (AexisCustomLayerRegistry.Register, CLR:160); Preflight()
// asks the library, for every HIP Gemm of a loaded session, whether a kernel
// exists at the activation rows the session will run, the question the
// reference's planner answers with missing-quantized-weight-only-kernel
// (TEP:389-407), and fails with every diagnostic at once.
using System;
using System.Collections.Generic;
using System.Text;
using Aexis.Execution;

namespace Aexis.Hip
{
    public sealed class AexisHipPlanException : InvalidOperationException
    {
        public AexisHipPlanException(IReadOnlyList<string> diagnostics)
            : base(Format(diagnostics))
        {
            Diagnostics = diagnostics;
        }

        public IReadOnlyList<string> Diagnostics { get; }

        static string Format(IReadOnlyList<string> diagnostics)
        {
            var sb = new StringBuilder("HIP quantized Gemm plan rejected | count=" + diagnostics.Count);
            foreach (var d in diagnostics)
                sb.Append("\n  ").Append(d);
            return sb.ToString();
        }
    }

    public static class AexisHipBackend
    {
        /// <summary>Routes `Gemm` layers to AexisHipGemmLayer when a HIP device and libaexq are
        /// present; returns false (and changes nothing) otherwise.</summary>
        public static bool Register()
        {
            if (!AexisHipDevice.Available())
                return false;
            try
            {
                if (Native.aexq_abi_version() != Aexq.AbiVersion)
                    return false;
            }
            catch (DllNotFoundException)
            {
                return false;
            }
            AexisHipGemmLayer.Register();
            return true;
        }

        /// <summary>Checks every HIP Gemm layer at each of `rows` (e.g. 1 for decode and the
        /// prompt length for prefill); throws AexisHipPlanException naming each layer and row
        /// count the library has no kernel for.</summary>
        public static void Preflight(AexisGraphSession owner, IEnumerable<AexisHipGemmLayer> layers,
                                     params int[] rows)
        {
            var bad = new List<string>();
            foreach (var layer in layers)
                foreach (var m in rows)
                {
                    var d = layer.PlanCheck(owner, m);
                    if (d != null)
                        bad.Add("rows=" + m + " | " + d);
                }
            if (bad.Count > 0)
                throw new AexisHipPlanException(bad);
        }
    }
}
