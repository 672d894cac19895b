"""CPU-side checks of the product: the C-ABI library loads and exports what
include/aexq.h declares, the host mirror's storage-shape rules match the
reference's, and the synthetic generators produce the stated formats.
No GPU call is made here."""
import ctypes

import numpy as np
import pytest

from aiimage_amd import _abi, synth


def test_library_loads_and_exports_every_header_symbol():
    lib = _abi.load()
    names = _abi.header_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert missing == []
    assert lib.aexq_abi_version() == 1
    assert isinstance(lib.aexq_last_error(), bytes)


def test_struct_layouts_match_header(tmp_path):
    """ctypes mirrors of the ABI structs have the C compiler's offsets and sizes."""
    import os
    import subprocess
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    probe = tmp_path / "probe.c"
    fields = {
        "aexq_tensor": (_abi.Tensor, ["logical", "storage", "layout", "dtype", "data", "batch",
                                      "batch_stride"]),
        "aexq_linear_args": (_abi.LinearArgs, ["alpha", "beta", "c", "broadcast_c", "rms_gamma",
                                               "rms_gamma_size", "rms_eps", "up", "residual",
                                               "flags"]),
        "aexq_weight_info": (_abi.WeightInfo, ["bits", "n", "k", "block", "scale_dtype",
                                               "nibble_code", "batch", "code_bytes",
                                               "scale_bytes"]),
    }
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "aexq.h"', "int main(void){"]
    for st, (_, names) in fields.items():
        lines.append(f'printf("{st} %zu\\n", sizeof({st}));')
        for f in names:
            lines.append(f'printf("{st}.{f} %zu\\n", offsetof({st}, {f}));')
    lines.append("return 0;}")
    probe.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-I", os.path.join(root, "include"), str(probe), "-o", str(exe)],
                   check=True)
    out = dict(l.split() for l in subprocess.run([str(exe)], capture_output=True, text=True,
                                                 check=True).stdout.splitlines())
    for st, (cls, names) in fields.items():
        assert int(out[st]) == ctypes.sizeof(cls), st
        for f in names:
            assert int(out[f"{st}.{f}"]) == getattr(cls, f).offset, (st, f)


def test_storage_shape_rules():
    from aiimage_amd import aexq
    # ResolvePack4LinearMatStorageShape (GS:10836-10841)
    assert aexq.pack4_linear_storage(3, 1024) == (3, 256, 3, 1, 4)
    assert aexq.pack4_linear_storage(1, 6) == (3, 2, 1, 1, 4)
    # ResolvePack4TiledLinearMatStorageShape (GS:10843-10852), LM head 151,936
    assert aexq.pack4_tiled_storage(1, 151936) == (3, 8192, 5, 1, 4)
    assert aexq.pack4_tiled_storage(8, 151936) == (3, 8192, 40, 1, 4)
    assert aexq.storage_elements(_abi.LAYOUT_PACK4_TILED, 1, 151936) == 8192 * 5 * 4
    assert aexq.storage_elements(_abi.LAYOUT_PACK4_LINEAR, 1, 6) == 8
    # GL:515-525 output storage choice
    assert aexq.output_layout_for(151936) == _abi.LAYOUT_PACK4_TILED
    assert aexq.output_layout_for(3584) == _abi.LAYOUT_PACK4_LINEAR
    assert aexq.output_layout_for(6) == _abi.LAYOUT_LINEAR


def test_make_args_flags():
    from aiimage_amd import aexq
    a = aexq.make_args(rmsnorm=True)
    assert a.flags == _abi.EPI_RMSNORM_IN
    assert a.alpha == 1.0 and a.beta == 1.0 and a.broadcast_c == -1


def test_synth_q8_format(orc):
    words, scales, codes = synth.q8_weights(64, 1024, seed=1)
    assert codes.min() >= -127 and codes.max() <= 127
    assert scales.dtype == np.float16
    # about 30% of |N(0,0.02)|/127 fall below the fp16 normal range
    sub = np.mean(np.abs(scales.astype(np.float32)) < 2.0 ** -14)
    assert 0.1 < sub < 0.5
    deq = orc.dequant_q8(words, scales, 64, 1024, scale_dtype=orc.SCALE_F16)
    assert np.array_equal(deq, codes.astype(np.float32) * scales.astype(np.float32)[:, None])


@pytest.mark.parametrize("code", [synth.NIBBLE_OFFSET8, synth.NIBBLE_TWOS])
def test_synth_q4_format(orc, code):
    words, scales, codes = synth.q4_weights(16, 256, seed=2, group=32, code=code)
    assert codes.min() >= -7 and codes.max() <= 7
    assert scales.size == 16 * 256 // 32
    deq = orc.dequant_q4(words, scales, 16, 256, 32, nibble_code=code, scale_dtype=orc.SCALE_F16)
    want = codes.astype(np.float32) * np.repeat(scales.astype(np.float32), 32).reshape(16, 256)
    assert np.array_equal(deq, want)
    # offset-8 stores q+8: an all-zero code row packs to 0x88888888 words
    z = synth.pack_nibbles(np.zeros((1, 8), np.int8), code)
    assert int(z[0]) == (0x88888888 if code == synth.NIBBLE_OFFSET8 else 0)


def test_archive_header_checks_match_the_reader(orc):
    """aexq_archive_header is host-only: it accepts what the oracle writer
    emits and rejects what NcnnQ8ArchiveReader rejects (Q8A:277-293)."""
    from aiimage_amd import aexq
    assert aexq.archive_header(orc.archive_header(4, 16, 7, 1 << 20)) == (4, 16, 7)
    assert aexq.archive_header(orc.archive_header(0, 256, 0, 0)) == (8, 256, 0)
    good = orc.archive_header(8, 64, 2, 99)
    bad_cases = [good[:31], b"\0" + good[1:], good[:8] + b"\2\0\0\0" + good[12:],
                 orc.archive_header(5, 64, 2, 99), orc.archive_header(8, 0, 2, 99),
                 orc.archive_header(8, 64, -1, 99)]
    for bad in bad_cases:
        with pytest.raises(_abi.InvalidDataError):
            aexq.archive_header(bad)


@pytest.mark.parametrize("head_dim,base,capacity", [(128, 1e6, 2048), (64, 1e7, 300)])
def test_decoder_rope_tables_equal_oracle_rows(orc, head_dim, base, capacity):
    """The decode session's [capacity][d/2] RoPE tables (built once on the host,
    indexed on the device by the decode position) hold, row for row and bit for
    bit, the oracle's table of that position, which the oracle tests pin
    against the frequency schedule and the rotation direction."""
    from aiimage_amd import decoder
    ct, st = decoder.rope_tables(capacity, head_dim, base)
    assert ct.shape == (capacity, head_dim // 2) and ct.dtype == np.float32
    for p in (0, 1, 2, 37, capacity // 2, capacity - 1):
        c, s = orc.rope_table(p, head_dim, base)
        assert np.array_equal(ct[p], c) and np.array_equal(st[p], s), p


def test_generate_argument_checks():
    """DecodeSession.generate refuses, before any device work, a graph_steps
    other than the captured graph's step count, a graph captured without
    advance, a step count below 1 and a run past the cache capacity (stand-in
    session and graph objects carry only what the checks read)."""
    from types import SimpleNamespace
    from aiimage_amd import decoder
    gen = decoder.DecodeSession.generate
    sess = SimpleNamespace(cfg=SimpleNamespace(capacity=64))
    four = SimpleNamespace(aexq_steps=4, aexq_advance=True)
    with pytest.raises(ValueError, match="graph of 4 steps"):
        gen(sess, 1, 0, 8, graph=four, graph_steps=2)
    with pytest.raises(ValueError, match="without advance"):
        gen(sess, 1, 0, 8, graph=SimpleNamespace(aexq_steps=2, aexq_advance=False))
    with pytest.raises(ValueError, match="graph_steps=0"):
        gen(sess, 1, 0, 8, graph_steps=0)
    with pytest.raises(ValueError, match="capacity"):
        gen(sess, 1, 60, 8, graph=four)


# ---------------------------------------------------------------- the C# binding


def _cs_dir():
    import os
    return os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "bindings", "csharp")


def _cs_structs():
    """{struct: (size, {field: offset})} of every [StructLayout(LayoutKind.Explicit,
    Size = N)] struct in bindings/csharp/*.cs, read from the source text."""
    import glob
    import re
    out = {}
    for path in sorted(glob.glob(_cs_dir() + "/*.cs")):
        text = open(path).read()
        for m in re.finditer(r"\[StructLayout\(LayoutKind\.Explicit, Size = (\d+)\)\]\s*public struct (\w+)\s*\{(.*?)\n    \}",
                             text, re.S):
            size, name, body = int(m.group(1)), m.group(2), m.group(3)
            fields = {f: int(o) for o, f in re.findall(r"\[FieldOffset\((\d+)\)\] public [\w\.]+ (\w+);", body)}
            out[name] = (size, fields)
    return out


def _snake(name: str) -> str:
    import re
    return re.sub(r"(?<=[a-z0-9])([A-Z])", r"_\1", name).lower()


# C# struct -> (C type, {C# field: C member}); members not listed map camelCase -> snake_case
_CS_TO_C = {
    "AexqShape": ("aexq_shape", {}),
    "AexqTensor": ("aexq_tensor", {}),
    "AexqLinearArgs": ("aexq_linear_args", {}),
    "AexqWeightInfo": ("aexq_weight_info", {}),
    "AexqDecoderLayer": ("aexq_decoder_layer", {}),
    "AexqDecoderConfig": ("aexq_decoder_config", {"attnScale": "attn_scale"}),
    "HipExternalMemoryHandleDesc": ("hipExternalMemoryHandleDesc",
                                    {"type": "type", "fd": "handle.fd", "win32Handle": "handle.win32.handle",
                                     "win32Name": "handle.win32.name", "size": "size", "flags": "flags"}),
    "HipExternalMemoryBufferDesc": ("hipExternalMemoryBufferDesc",
                                    {"offset": "offset", "size": "size", "flags": "flags"}),
    "HipExternalSemaphoreHandleDesc": ("hipExternalSemaphoreHandleDesc",
                                       {"type": "type", "fd": "handle.fd", "win32Handle": "handle.win32.handle",
                                        "win32Name": "handle.win32.name", "flags": "flags"}),
    "HipExternalSemaphoreParams": ("hipExternalSemaphoreSignalParams",
                                   {"fenceValue": "params.fence.value", "flags": "flags"}),
}


def test_csharp_struct_offsets_match_the_c_compiler(tmp_path):
    """Every explicit-layout struct of the C# binding has the C compiler's size and
    member offsets (aexq.h, and hip_runtime_api.h for the external-memory imports;
    the semaphore wait parameters share the signal parameters' layout)."""
    import os
    import subprocess
    cs = _cs_structs()
    assert set(cs) == set(_CS_TO_C), sorted(set(cs) ^ set(_CS_TO_C))
    lines = ["#include <stdio.h>", "#include <stddef.h>", "#include <hip/hip_runtime_api.h>",
             '#include "aexq.h"', "int main(void){"]
    for name, (ctype, names) in _CS_TO_C.items():
        lines.append(f'printf("{name} %zu\\n", sizeof({ctype}));')
        for f in cs[name][1]:
            member = names.get(f, _snake(f))
            lines.append(f'printf("{name}.{f} %zu\\n", offsetof({ctype}, {member}));')
    lines.append('printf("wait %zu %zu %zu\\n", sizeof(hipExternalSemaphoreWaitParams), '
                 'offsetof(hipExternalSemaphoreWaitParams, params.fence.value), '
                 'offsetof(hipExternalSemaphoreWaitParams, flags));')
    lines.append("return 0;}")
    probe = tmp_path / "cs_probe.c"
    probe.write_text("\n".join(lines))
    exe = tmp_path / "cs_probe"
    root = os.path.dirname(_cs_dir().rstrip("/").rsplit("/", 1)[0])
    subprocess.run(["gcc", "-D__HIP_PLATFORM_AMD__", "-I", "/opt/rocm/include", "-I",
                    os.path.join(root, "include"), str(probe), "-o", str(exe)], check=True)
    got = {}
    for line in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines():
        k, *v = line.split()
        got[k] = [int(x) for x in v]
    for name, (size, fields) in cs.items():
        assert got[name] == [size], (name, got[name], size)
        for f, off in fields.items():
            assert got[f"{name}.{f}"] == [off], (name, f, got[f"{name}.{f}"], off)
    assert got["wait"] == [cs["HipExternalSemaphoreParams"][0], 0, cs["HipExternalSemaphoreParams"][1]["flags"]]


def test_csharp_binding_imports_every_header_function():
    """bindings/csharp/Native.cs has a DllImport for every function include/aexq.h
    declares, with the C parameter count, and none the header lacks."""
    import re
    text = open(_cs_dir() + "/Native.cs").read()
    imports = {}
    for m in re.finditer(r"\[DllImport\(Lib(?:, EntryPoint = \"(\w+)\")?\)\] public static extern [\w\.]+ (\w+)\((.*?)\);",
                         text, re.S):
        entry = m.group(1) or m.group(2)
        params = re.sub(r"/\*.*?\*/", "", m.group(3)).strip()
        imports.setdefault(entry, set()).add(0 if not params else params.count(",") + 1)
    header = open(_cs_dir().rsplit("/", 2)[0] + "/include/aexq.h").read()
    header = re.sub(r"/\*.*?\*/", "", header, flags=re.S)
    decls = {}
    for m in re.finditer(r"^(?:aexq_status|void|int|const char\*)\s+(aexq_\w+)\((.*?)\);", header, re.S | re.M):
        params = m.group(2).strip()
        decls[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    assert set(decls) == set(_abi.header_functions())
    assert set(imports) == set(decls), sorted(set(imports) ^ set(decls))
    for name, n in decls.items():
        assert imports[name] == {n}, (name, imports[name], n)
