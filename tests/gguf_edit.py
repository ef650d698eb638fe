"""Reads and rewrites GGUF v3 files for the load-error tests: the metadata is
kept as raw bytes, the tensor table is parsed so that a tensor can be dropped
or given another shape, and the data section is copied unchanged (tensor
offsets are relative to its start, which is re-aligned after the table)."""

import struct

_SCALAR = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 7: 1, 10: 8, 11: 8, 12: 8}  # GGUF value type -> bytes


class Gguf:
    def __init__(self, data: bytes):
        self.data = data
        i = 0
        self.magic, self.version, n_tensors, n_kv = struct.unpack_from("<4sIQQ", data, i)
        i += 24
        kv_start = i
        self.alignment = 32
        for _ in range(n_kv):
            key, i = self._string(i)
            (vtype,) = struct.unpack_from("<I", data, i)
            i += 4
            if key == "general.alignment" and vtype == 4:
                (self.alignment,) = struct.unpack_from("<I", data, i)
            i = self._skip_value(i, vtype)
        self.n_kv = n_kv
        self.kv = data[kv_start:i]
        self.tensors = []  # [name, dims, type, offset]
        for _ in range(n_tensors):
            name, i = self._string(i)
            (nd,) = struct.unpack_from("<I", data, i)
            i += 4
            dims = list(struct.unpack_from(f"<{nd}Q", data, i))
            i += 8 * nd
            ttype, off = struct.unpack_from("<IQ", data, i)
            i += 12
            self.tensors.append([name, dims, ttype, off])
        self.body = data[(i + self.alignment - 1) // self.alignment * self.alignment:]

    def _string(self, i):
        (n,) = struct.unpack_from("<Q", self.data, i)
        return self.data[i + 8:i + 8 + n].decode(), i + 8 + n

    def _skip_value(self, i, vtype):
        if vtype == 8:
            (n,) = struct.unpack_from("<Q", self.data, i)
            return i + 8 + n
        if vtype == 9:
            etype, count = struct.unpack_from("<IQ", self.data, i)
            i += 12
            for _ in range(count):
                i = self._skip_value(i, etype)
            return i
        return i + _SCALAR[vtype]

    def names(self):
        return [t[0] for t in self.tensors]

    def drop(self, name):
        self.tensors = [t for t in self.tensors if t[0] != name]

    def reshape(self, name, dims):
        for t in self.tensors:
            if t[0] == name:
                t[1] = list(dims)

    def dump(self) -> bytes:
        out = bytearray(struct.pack("<4sIQQ", self.magic, self.version, len(self.tensors), self.n_kv))
        out += self.kv
        for name, dims, ttype, off in self.tensors:
            b = name.encode()
            out += struct.pack("<Q", len(b)) + b + struct.pack("<I", len(dims))
            out += struct.pack(f"<{len(dims)}Q", *dims) + struct.pack("<IQ", ttype, off)
        out += b"\0" * ((-len(out)) % self.alignment)
        return bytes(out) + self.body
