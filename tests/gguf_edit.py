"""A small GGUF v3 reader/writer for tests: parse a file into its metadata bytes, tensor infos
and data section, change tensor infos (extents, offsets, types) or a tensor's payload bytes, and
write a new file."""
import struct

_SCALAR = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 7: 1, 10: 8, 11: 8, 12: 8}


def _skip_value(b, p, t):
    if t == 8:
        (n,) = struct.unpack_from("<Q", b, p)
        return p + 8 + n
    if t == 9:
        et, n = struct.unpack_from("<IQ", b, p)
        p += 12
        for _ in range(n):
            p = _skip_value(b, p, et)
        return p
    return p + _SCALAR[t]


class Gguf:
    def __init__(self, path):
        b = open(path, "rb").read()
        magic, self.version, nt, nkv = struct.unpack_from("<IIQQ", b, 0)
        assert magic == 0x46554747
        p = 24
        kv0 = p
        self.alignment = 32
        for _ in range(nkv):
            (n,) = struct.unpack_from("<Q", b, p)
            key = b[p + 8:p + 8 + n].decode()
            p += 8 + n
            (t,) = struct.unpack_from("<I", b, p)
            p += 4
            if key == "general.alignment":
                (self.alignment,) = struct.unpack_from("<I", b, p)
            p = _skip_value(b, p, t)
        self.nkv, self.kv_bytes = nkv, b[kv0:p]
        self.tensors = []
        for _ in range(nt):
            (n,) = struct.unpack_from("<Q", b, p)
            name = b[p + 8:p + 8 + n].decode()
            p += 8 + n
            (nd,) = struct.unpack_from("<I", b, p)
            ne = list(struct.unpack_from(f"<{nd}Q", b, p + 4))
            p += 4 + 8 * nd
            t, off = struct.unpack_from("<IQ", b, p)
            p += 12
            self.tensors.append({"name": name, "ne": ne, "type": t, "offset": off})
        a = self.alignment
        self.data = b[(p + a - 1) // a * a:]

    def tensor(self, name):
        return next(t for t in self.tensors if t["name"] == name)

    _BLOCK = {0: (1, 4), 1: (1, 2), 2: (32, 18), 8: (32, 34), 12: (256, 144), 13: (256, 176),
              14: (256, 210)}

    def nbytes(self, name):
        t = self.tensor(name)
        n = 1
        for v in t["ne"]:
            n *= v
        bs, tb = self._BLOCK[t["type"]]
        return n // bs * tb

    def payload(self, name):
        t = self.tensor(name)
        return self.data[t["offset"]:t["offset"] + self.nbytes(name)]

    def set_payload(self, name, raw):
        """Replace a tensor's bytes (same length)."""
        t = self.tensor(name)
        raw = bytes(raw)
        assert len(raw) == self.nbytes(name)
        d = bytearray(self.data)
        d[t["offset"]:t["offset"] + len(raw)] = raw
        self.data = bytes(d)

    def zero(self, name):
        """All-zero payload: every k-quant block with d = dmin = 0, i.e. an all-zero matrix."""
        self.set_payload(name, b"\0" * self.nbytes(name))

    def write(self, path):
        out = bytearray(struct.pack("<IIQQ", 0x46554747, self.version, len(self.tensors), self.nkv))
        out += self.kv_bytes
        for t in self.tensors:
            nm = t["name"].encode()
            out += struct.pack("<Q", len(nm)) + nm + struct.pack("<I", len(t["ne"]))
            out += struct.pack(f"<{len(t['ne'])}Q", *[v & 0xFFFFFFFFFFFFFFFF for v in t["ne"]])
            out += struct.pack("<IQ", t["type"], t["offset"] & 0xFFFFFFFFFFFFFFFF)
        a = self.alignment
        out += b"\0" * ((-len(out)) % a)
        out += self.data
        open(path, "wb").write(bytes(out))
        return path
