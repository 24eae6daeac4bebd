"""Kernel metadata of the gfx950 code objects inside the in-tree library.

The library's `.hip_fatbin` section holds one clang offload bundle per HIP
source; each bundle's gfx950 entry is an AMDGPU ELF code object whose
NT_AMDGPU_METADATA note (a msgpack map) lists every kernel with its resource
use (`.private_segment_fixed_size`, `.vgpr_count`, ...). Only the library
built here from this repository's sources is read.
"""

from __future__ import annotations

import struct
from pathlib import Path

import msgpack

_BUNDLE_MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
_NT_AMDGPU_METADATA = 32
_SHT_NOTE = 7


def _sections(elf: bytes) -> list[tuple[str, int, int, int]]:
    """(name, type, offset, size) of every section of a 64-bit little-endian ELF."""
    assert elf[:4] == b"\x7fELF" and elf[4] == 2 and elf[5] == 1, "not a 64-bit little-endian ELF"
    shoff, = struct.unpack_from("<Q", elf, 0x28)
    shentsize, shnum, shstrndx = struct.unpack_from("<HHH", elf, 0x3A)
    heads = [struct.unpack_from("<IIQQQQIIQQ", elf, shoff + i * shentsize) for i in range(shnum)]
    str_off, str_size = heads[shstrndx][4], heads[shstrndx][5]
    names = elf[str_off:str_off + str_size]
    out = []
    for h in heads:
        name = names[h[0]:names.index(b"\0", h[0])].decode()
        out.append((name, h[1], h[4], h[5]))
    return out


def _bundle_entries(blob: bytes, start: int) -> list[tuple[str, bytes]]:
    n, = struct.unpack_from("<Q", blob, start + len(_BUNDLE_MAGIC))
    pos = start + len(_BUNDLE_MAGIC) + 8
    entries = []
    for _ in range(n):
        off, size, tlen = struct.unpack_from("<QQQ", blob, pos)
        triple = blob[pos + 24:pos + 24 + tlen].decode()
        pos += 24 + tlen
        entries.append((triple, blob[start + off:start + off + size]))
    return entries


def _metadata_kernels(code_object: bytes) -> list[dict]:
    kernels = []
    for _name, stype, off, size in _sections(code_object):
        if stype != _SHT_NOTE:
            continue
        pos, end = off, off + size
        while pos + 12 <= end:
            namesz, descsz, ntype = struct.unpack_from("<III", code_object, pos)
            name = code_object[pos + 12:pos + 12 + namesz].rstrip(b"\0")
            desc_at = pos + 12 + ((namesz + 3) & ~3)
            if ntype == _NT_AMDGPU_METADATA and name == b"AMDGPU":
                meta = msgpack.unpackb(code_object[desc_at:desc_at + descsz], raw=False, strict_map_key=False)
                kernels.extend(meta.get("amdhsa.kernels", []))
            pos = desc_at + ((descsz + 3) & ~3)
    return kernels


def gfx950_kernels(library: Path) -> list[dict]:
    """Metadata maps of every gfx950 kernel in the library's offload bundles."""
    lib = Path(library).read_bytes()
    fatbin = next((off, size) for name, _t, off, size in _sections(lib) if name == ".hip_fatbin")
    blob = lib[fatbin[0]:fatbin[0] + fatbin[1]]
    kernels = []
    at = blob.find(_BUNDLE_MAGIC)
    while at >= 0:
        for triple, code_object in _bundle_entries(blob, at):
            if triple.endswith("gfx950"):
                kernels.extend(_metadata_kernels(code_object))
        at = blob.find(_BUNDLE_MAGIC, at + 1)
    return kernels
