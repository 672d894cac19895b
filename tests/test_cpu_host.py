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
