"""Kernel descriptors of the built library (CPU only; reads the gfx950 code objects
embedded in libmoe_mi355x.so, which this repository builds from its own sources).

Guards against code-generation regressions that cost time without changing results:
  * no kernel may request the dispatch-packet or queue pointer. A kernel that does
    reads the dispatch packet in every wave at its start; the combine kernel once did
    (a small int array that the compiler placed in LDS, whose per-thread addressing
    needs the workgroup size from the packet), which held each workgroup 3-12 us;
  * no kernel uses scratch memory except the prefill GEMM2 loader kernel's 16 bytes of
    register spill (a stack array or a larger spill would show here first);
  * the combine kernel uses no LDS at all.
The descriptor is the 64-byte AMDHSA kernel descriptor (symbol `<kernel>.kd`): group
segment size at byte 0, private segment size at byte 4, kernel code properties at byte
56 (bit 1: dispatch pointer, bit 2: queue pointer)."""
import os
import struct

import pytest

from flashinfer_mlsys_amd import _lib

BUNDLE_MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
EXPECTED = ("route_kernel", "route_count_kernel", "dispatch_count_kernel", "dispatch_scatter_kernel",
            "dispatch_small_kernel", "gemm1_decode_kernel", "gemm2_decode_kernel", "gemm1_prefill_kernel",
            "gemm2_loader_kernel", "combine_kernel", "quantize_1x128_kernel", "router_small_kernel",
            "router_tiled_kernel", "router_ksplit_kernel")
SCRATCH_ALLOWED = {"gemm2_loader_kernel": 64}


def _cstr(buf, off):
    return buf[off:buf.index(b"\0", off)].decode()


def _sections(elf):
    shoff, = struct.unpack_from("<Q", elf, 0x28)
    shentsize, shnum, shstrndx = struct.unpack_from("<HHH", elf, 0x3A)
    secs = []
    for i in range(shnum):
        name, typ, _flags, addr, off, size, link, _info, _align, _ent = struct.unpack_from(
            "<IIQQQQIIQQ", elf, shoff + i * shentsize)
        secs.append({"name": name, "type": typ, "addr": addr, "off": off, "size": size, "link": link})
    for s in secs:
        s["sname"] = _cstr(elf, secs[shstrndx]["off"] + s["name"])
    return secs


def _kernel_descriptors(co):
    """{kernel symbol: (group segment bytes, private segment bytes, code properties)}"""
    secs = _sections(co)
    out = {}
    for s in secs:
        if s["type"] != 2:  # SHT_SYMTAB
            continue
        strs = secs[s["link"]]
        for k in range(s["size"] // 24):
            st_name, _info, _other, shndx, value, _size = struct.unpack_from("<IBBHQQ", co, s["off"] + 24 * k)
            name = _cstr(co, strs["off"] + st_name)
            if name.endswith(".kd") and 0 < shndx < len(secs):
                sec = secs[shndx]
                d = co[sec["off"] + value - sec["addr"]:][:64]
                lds, priv = struct.unpack_from("<II", d, 0)
                props, = struct.unpack_from("<H", d, 56)
                out[name[:-3]] = (lds, priv, props)
    return out


def library_descriptors(path):
    so = open(path, "rb").read()
    fatbin = [s for s in _sections(so) if s["sname"] == ".hip_fatbin"]
    assert fatbin, "no device code section in the library"
    data = so[fatbin[0]["off"]:fatbin[0]["off"] + fatbin[0]["size"]]
    out = {}
    pos = data.find(BUNDLE_MAGIC)
    while pos >= 0:  # one offload bundle per source file
        n, = struct.unpack_from("<Q", data, pos + 24)
        p = pos + 32
        for _ in range(n):
            off, size, tlen = struct.unpack_from("<QQQ", data, p)
            triple = data[p + 24:p + 24 + tlen].decode()
            p += 24 + tlen
            if "gfx950" in triple:
                out.update(_kernel_descriptors(data[pos + off:pos + off + size]))
        pos = data.find(BUNDLE_MAGIC, pos + 32)
    return out


def _short(symbol):
    for k in EXPECTED:
        if k in symbol:
            return k
    return symbol


@pytest.fixture(scope="module")
def descriptors():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libmoe_mi355x.so is not built: run python -m flashinfer_mlsys_amd.build")
    return library_descriptors(_lib.LIB_PATH)


def test_every_kernel_found(descriptors):
    found = {_short(s) for s in descriptors}
    assert set(EXPECTED) <= found, sorted(set(EXPECTED) - found)


def test_no_dispatch_or_queue_pointer(descriptors):
    bad = [_short(s) for s, (_lds, _priv, props) in descriptors.items() if props & 0b110]
    assert not bad, f"kernels reading the dispatch packet or queue: {bad}"


def test_scratch(descriptors):
    bad = {_short(s): priv for s, (_lds, priv, _props) in descriptors.items()
           if priv > SCRATCH_ALLOWED.get(_short(s), 0)}
    assert not bad, f"private segment bytes per lane: {bad}"


def test_combine_uses_no_lds(descriptors):
    lds = [lds for s, (lds, _priv, _props) in descriptors.items() if _short(s) == "combine_kernel"]
    assert lds == [0]
