"""CPU tests of the microbenchmark library behind ``bench.py --probes``: it
loads, and every entry point refuses sizes it would read or write out of
bounds before launching anything (no GPU is touched here)."""
from __future__ import annotations

import importlib

from conftest import PKG  # noqa: F401  (registers the package)

P = importlib.import_module("inference_systems_amd.probes")


def test_probe_library_loads_with_every_entry_point():
    lib = P.load()
    for name in P._SIGS:
        assert hasattr(lib, name), name


def test_probes_refuse_unsafe_sizes_before_launch():
    lib = P.load()
    assert lib.nvprobe_empty(0, None) == -1
    # the buffer must be exactly workgroups x 256 lanes x loads x 16 bytes
    assert lib.nvprobe_stream_read(None, 4096 * 16 + 16, 16, 1, None, None, None) == -1
    assert lib.nvprobe_stream_read(None, 4096 * 16, 16, 3, None, None, None) == -1
    assert lib.nvprobe_stream_read(None, 0, 0, 1, None, None, None) == -1
    assert lib.nvprobe_lds_read(256, 12, None, None, None) == -1
    assert lib.nvprobe_lds_read(0, 16, None, None, None) == -1
    # copy window: a positive multiple of 1 KiB; in-flight 8 or 16; iterations a multiple of it
    fake = 1 << 20   # never dereferenced: every call below is refused first
    assert lib.nvprobe_copy(0, None, 4096, 256, 64, 8, 0, fake, None, None) == -1
    assert lib.nvprobe_copy(0, fake, 4096, 256, 64, 8, 0, None, None, None) == -1
    assert lib.nvprobe_copy(0, fake, 1000, 256, 64, 8, 0, fake, None, None) == -1
    assert lib.nvprobe_copy(0, fake, 4096, 256, 64, 4, 0, fake, None, None) == -1
    assert lib.nvprobe_copy(0, fake, 4096, 256, 60, 8, 0, fake, None, None) == -1
    assert lib.nvprobe_copy(0, fake, 4096, 256, 64, 8, 2, fake, None, None) == -1
    assert lib.nvprobe_copy(4, fake, 4096, 256, 64, 8, 0, fake, None, None) == -1
    assert lib.nvprobe_mfma(256, 16, 3, None, None, None) == -1
    assert lib.nvprobe_mfma16(256, 16, 2, None, None, None) == -1
    assert lib.nvprobe_mfma16(0, 16, 4, None, None, None) == -1
    # LDS lane map: offsets inside the 16 KiB region and aligned to the width
    import ctypes
    fake_sink = 1 << 20
    ok = (ctypes.c_uint32 * 64)(*[lane * 256 for lane in range(64)])
    high = (ctypes.c_uint32 * 64)(*([lane * 256 for lane in range(63)] + [16384 - 8]))
    odd = (ctypes.c_uint32 * 64)(*([4] + [lane * 256 for lane in range(1, 64)]))
    assert lib.nvprobe_lds_map(high, 16, 0, 256, 64, fake_sink, fake_sink, None) == -1
    assert lib.nvprobe_lds_map(odd, 8, 0, 256, 64, fake_sink, fake_sink, None) == -1
    assert lib.nvprobe_lds_map(ok, 12, 0, 256, 64, fake_sink, fake_sink, None) == -1
    assert lib.nvprobe_lds_map(ok, 16, 2, 256, 64, fake_sink, fake_sink, None) == -1
    assert lib.nvprobe_lds_map(ok, 16, 0, 256, 60, fake_sink, fake_sink, None) == -1
    assert lib.nvprobe_lds_map(ok, 16, 0, 0, 64, fake_sink, fake_sink, None) == -1
    assert lib.nvprobe_lds_map(None, 16, 0, 256, 64, fake_sink, fake_sink, None) == -1
    # each 128-row tile writes 512 bytes per row: ld must cover tiles_n of them
    assert lib.nvprobe_write_tiles(None, 8192 - 16, 16, 16, 1, None, None) == -1
    assert lib.nvprobe_write_tiles(None, 8192 + 8, 16, 16, 1, None, None) == -1


def test_decode_sweep_library_lists_and_refuses():
    """The decode configuration sweep: every configuration has a name and an
    A-row limit; launches with a bad configuration, null pointers, M above
    the configuration's rows or K not a multiple of 8 are refused before
    anything is launched."""
    cfgs = P.sweep_configs()
    assert len(cfgs) >= 10
    names = [name for _, name, _, _ in cfgs]
    assert len(set(names)) == len(names)
    assert all(name.split()[0] in ("lds", "areg", "lines", "kn") for name in names)
    assert all(kn == (name.split()[0] == "kn") for _, name, _, kn in cfgs)
    assert {rows for _, _, rows, _ in cfgs} == {8, 16, 32}
    lib = P.load_sweep()
    fake = 1 << 20   # never dereferenced: every call below is refused first
    assert lib.nvsweep_decode(-1, fake, fake, fake, 1, 64, 64, None) == -1
    assert lib.nvsweep_decode(len(cfgs), fake, fake, fake, 1, 64, 64, None) == -1
    assert lib.nvsweep_decode(0, None, fake, fake, 1, 64, 64, None) == -1
    idx8 = next(i for i, _, rows, kn in cfgs if rows == 8 and not kn)
    idx_kn = next(i for i, _, rows, kn in cfgs if rows == 8 and kn)
    assert lib.nvsweep_decode(idx_kn, fake, fake, fake, 1, 60, 64, None) == -1   # N not a multiple of 8
    assert lib.nvsweep_decode(idx8, fake, fake, fake, 9, 64, 64, None) == -1
    assert lib.nvsweep_decode(idx8, fake, fake, fake, 1, 64, 60, None) == -1
    assert lib.nvsweep_decode(idx8, fake, fake, fake, 0, 64, 64, None) == -1
    assert lib.nvsweep_decode_name(len(cfgs)) == b""
    assert lib.nvsweep_decode_kn(len(cfgs)) == -1
