"""A small GGUF v3 writer and reader for the loader tests (test infrastructure).

Images are built from metadata key/values and tensors (name, dims, GGML type id, raw bytes) in
the layout gguf::read_file (src/gguf.rs:454-551) parses: magic, version, counts, metadata,
tensor infos, data aligned to general.alignment (default 32)."""
import struct

import numpy as np

T_U32, T_I32, T_F32, T_STR, T_ARR, T_U64 = 4, 5, 6, 8, 9, 10


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _val(t: int, v) -> bytes:
    if t == T_U32:
        return struct.pack("<I", v)
    if t == T_I32:
        return struct.pack("<i", v)
    if t == T_F32:
        return struct.pack("<f", v)
    if t == T_U64:
        return struct.pack("<Q", v)
    if t == T_STR:
        return _str(v)
    if t == T_ARR:  # v = (item type, items)
        it, items = v
        return struct.pack("<I", it) + struct.pack("<Q", len(items)) + b"".join(_val(it, x) for x in items)
    raise ValueError(t)


def write(meta, tensors, alignment=32, data=True) -> bytes:
    """meta: [(key, type, value)]; tensors: [(name, dims, ggml_type, bytes)] (bytes may be
    shorter than the tensor when data=False: a header-only image)."""
    h = bytearray(b"GGUF" + struct.pack("<I", 3) + struct.pack("<Q", len(tensors)) + struct.pack("<Q", len(meta)))
    for k, t, v in meta:
        h += _str(k) + struct.pack("<I", t) + _val(t, v)
    off = 0
    offsets = []
    for name, dims, ty, raw in tensors:
        offsets.append(off)
        h += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        h += struct.pack("<I", ty) + struct.pack("<Q", off)
        off += (len(raw) + alignment - 1) // alignment * alignment
    start = (len(h) + alignment - 1) // alignment * alignment
    h += b"\0" * (start - len(h))
    if not data:
        return bytes(h)
    body = bytearray(off)
    for (name, dims, ty, raw), o in zip(tensors, offsets):
        body[o:o + len(raw)] = raw
    return bytes(h + body)


def read(img: bytes):
    """Minimal parse back into (meta [(key, type, value)], tensors [(name, dims, type, bytes)])
    for images whose metadata uses only the scalar and string types above (the synthetic
    writer's); the tensor bytes run to the next tensor's offset or the end of the file."""
    pos = 0

    def u(n):
        nonlocal pos
        v = int.from_bytes(img[pos:pos + n], "little")
        pos += n
        return v

    def s():
        n = u(8)
        nonlocal pos
        r = img[pos:pos + n].decode()
        pos += n
        return r

    assert img[:4] == b"GGUF"
    pos = 4
    u(4)
    nt, nm = u(8), u(8)
    meta = []
    for _ in range(nm):
        k, t = s(), u(4)
        if t == T_STR:
            v = s()
        elif t == T_F32:
            v = struct.unpack("<f", img[pos:pos + 4])[0]
            pos += 4
        elif t in (T_U32, T_I32):
            v = u(4)
            if t == T_I32 and v >= 1 << 31:
                v -= 1 << 32
        elif t == T_U64:
            v = u(8)
        else:
            raise ValueError(f"metadata type {t} not handled")
        meta.append((k, t, v))
    infos = []
    for _ in range(nt):
        name = s()
        nd = u(4)
        dims = [u(8) for _ in range(nd)]
        infos.append((name, dims, u(4), u(8)))
    start = (pos + 31) // 32 * 32
    tensors = [(name, dims, ty, img[start + o:start + o + nbytes(dims, ty)]) for name, dims, ty, o in infos]
    return meta, tensors


LAYOUT = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34), 12: (256, 144),
          13: (256, 176), 14: (256, 210), 30: (1, 2)}


def _f16(rng, n, lo=1e-3, hi=2e-2):
    return rng.uniform(lo, hi, n).astype(np.float16).view(np.uint16)


def random_blocks(ty, nblk, seed):
    rng = np.random.default_rng(seed)
    bs, tsz = LAYOUT[ty]
    if ty == 0:
        return rng.normal(0, 1, nblk).astype(np.float32).view(np.uint8)
    if ty == 1:
        return rng.normal(0, 1, nblk).astype(np.float16).view(np.uint8)
    if ty == 30:
        return (rng.normal(0, 1, nblk).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16).view(np.uint8)
    b = rng.integers(0, 256, (nblk, tsz), dtype=np.uint8)
    if ty in (2, 3, 6, 7, 8):
        b[:, 0:2] = _f16(rng, nblk).view(np.uint8).reshape(nblk, 2)
        if ty in (3, 7):
            b[:, 2:4] = _f16(rng, nblk, -0.1, 0.1).view(np.uint8).reshape(nblk, 2)
    elif ty in (12, 13):
        b[:, 0:2] = _f16(rng, nblk).view(np.uint8).reshape(nblk, 2)
        b[:, 2:4] = _f16(rng, nblk).view(np.uint8).reshape(nblk, 2)
    elif ty == 14:
        b[:, 208:210] = _f16(rng, nblk).view(np.uint8).reshape(nblk, 2)
    return b.ravel()



def q6_k_weights(nblk, seed, std=0.02):
    """Random Q6_K blocks whose elements d * scale * (q - 32) have a standard deviation near
    std (random 6-bit values, scales in [-24, 24], d set from std), like a quantised N(0, std)
    weight matrix rather than random_blocks' full-range scales."""
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, (nblk, 210), dtype=np.uint8)
    b[:, 192:208] = rng.integers(-24, 25, (nblk, 16)).astype(np.int8).view(np.uint8)
    d = rng.uniform(0.6, 1.4, nblk) * std / (18.5 * 14.1)  # std of (q - 32) and of the scales
    b[:, 208:210] = d.astype(np.float16).view(np.uint8).reshape(nblk, 2)
    return b.ravel()


def with_types(image, types, seed=0):
    """The GGUF image with the named matrices replaced by random blocks of another type
    (Q6_K: q6_k_weights; Q4_0: random_blocks), the way llama.cpp's Q4_K_M recipe keeps some
    attn_v / ffn_down matrices in Q6_K."""
    meta, ts = read(bytes(image))
    out = []
    for i, (n, dims, ty, raw) in enumerate(ts):
        if n in types:
            ty = types[n]
            nblk = int(np.prod(dims)) // LAYOUT[ty][0]
            raw = (q6_k_weights(nblk, seed + i) if ty == 14 else random_blocks(ty, nblk, seed + i)).tobytes()
        out.append((n, dims, ty, raw))
    return write(meta, out)


def nbytes(dims, ty) -> int:
    bs, ts = LAYOUT[ty]
    return int(np.prod(dims)) // bs * ts
