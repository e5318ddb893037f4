"""The .walsh v4 model file on the GPU.

``load_walsh`` reads what compress.py writes (compress.py:140-360; the
reference reader is generate_compressed.py:118-270) and ``save_walsh``
writes it:

    b'SPIN', u16 version (4), u32 length + config JSON, then chunks
    marker (1 byte), u16 length + name (UTF-8), payload; b'END!' last.

Payloads (little-endian): an array is u8 dtype code (0 int8, 1 int32,
2 float16, 3 float32), u8 ndim, u32 dims, raw data.
    E / A  f32 scale + int8 array  (embedding / hash table = data * scale)
    B      u8 ndim, u32 dims, u32 num_nonzero, u32 length + bitmask bytes,
           u32 length + sign bytes (ternary Hadamard/octonion weights)
    S L N H h I   float16 array (beta, alpha, norm, head mixer W / beta,
           hash importance); R float32 [..., 2] array (RoPE, complex);
           J int32 array.

The bitmask + sign tensors are decoded on the GPU (walsh_ternary_from_bitmask),
either to the float codes the reference loader returns or, with
``packed_ternary=True``, straight into the 2-bit packed buffers
(pack_ternary_weights layout) that HadamardPackedLinear / OctonionPackedLinear
hold.  The file itself is parsed on the host (it is I/O, not compute).
"""
import json
import struct

import numpy as np
import torch

from .model import kernels

MAGIC = b'SPIN'
VERSION = 4
_DTYPES = {0: np.int8, 1: np.int32, 2: np.float16, 3: np.float32}
_CODES = {np.dtype(np.int8): 0, np.dtype(np.int32): 1, np.dtype(np.float16): 2, np.dtype(np.float32): 3}
_TERNARY_KEYS = ('wq', 'wk', 'wv', 'wo', 'gate_proj', 'up_proj', 'down_proj')


class _Reader:
    def __init__(self, buf: bytes):
        self.buf = memoryview(buf)
        self.pos = 0

    def take(self, n: int) -> memoryview:
        if self.pos + n > len(self.buf):
            raise ValueError(f".walsh file truncated at byte {self.pos} (needs {n} more)")
        v = self.buf[self.pos:self.pos + n]
        self.pos += n
        return v

    def u8(self):
        return struct.unpack('<B', self.take(1))[0]

    def u16(self):
        return struct.unpack('<H', self.take(2))[0]

    def u32(self):
        return struct.unpack('<I', self.take(4))[0]

    def f32(self):
        return struct.unpack('<f', self.take(4))[0]

    def name(self) -> str:
        return bytes(self.take(self.u16())).decode('utf-8')

    def array(self) -> np.ndarray:
        code = self.u8()
        if code not in _DTYPES:
            raise ValueError(f".walsh array with unknown dtype code {code}")
        shape = tuple(self.u32() for _ in range(self.u8()))
        dt = np.dtype(_DTYPES[code])
        n = int(np.prod(shape)) * dt.itemsize
        return np.frombuffer(bytes(self.take(n)), dtype=dt).reshape(shape)


def _to_device(a: np.ndarray, device) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if not a.flags.writeable:       # views of the file buffer: torch wants writable memory
        a = a.copy()
    return torch.from_numpy(a).to(device)


def load_walsh(path: str, device='cuda', packed_ternary: bool = False):
    """(state_dict, config) of a .walsh v4 file.  Tensors land on ``device``
    (a GPU: the ternary decode runs there).  Ternary weights are float32
    codes {-1, 0, 1} of the stored shape, or uint8 packed codes
    [..., ceil(K/4)] with ``packed_ternary``."""
    device = torch.device(device)
    if device.type != 'cuda':
        raise RuntimeError("load_walsh decodes on the GPU; pass a cuda device")
    with open(path, 'rb') as f:
        r = _Reader(f.read())
    if bytes(r.take(4)) != MAGIC:
        raise ValueError(f"{path}: not a .walsh file (bad magic)")
    version = r.u16()
    if version != VERSION:
        raise ValueError(f"{path}: .walsh version {version}; this loader reads version {VERSION}")
    config = json.loads(bytes(r.take(r.u32())).decode('utf-8'))
    sd = {}
    while r.pos < len(r.buf):
        marker = bytes(r.take(1))
        if marker == b'\x00':
            break
        if marker == b'E' and bytes(r.buf[r.pos:r.pos + 3]) == b'ND!':
            r.pos += 3
            break
        name = r.name()
        if marker in (b'E', b'A'):
            scale = r.f32()
            q = _to_device(r.array(), device)
            sd[name] = q.to(torch.float32) * scale
        elif marker == b'B':
            shape = tuple(r.u32() for _ in range(r.u8()))
            nnz = r.u32()
            bm = np.frombuffer(bytes(r.take(r.u32())), dtype=np.uint8)
            sg = np.frombuffer(bytes(r.take(r.u32())), dtype=np.uint8)
            out = kernels.ternary_from_bitmask(_to_device(bm, device), _to_device(sg, device), nnz, shape,
                                               packed=packed_ternary, codes=not packed_ternary)
            sd[name] = out['packed'] if packed_ternary else out['codes'].to(torch.float32)
        elif marker in (b'S', b'L', b'N', b'H', b'h', b'I'):
            sd[name] = _to_device(r.array(), device).to(torch.float32)
        elif marker == b'R':
            sd[name] = torch.view_as_complex(_to_device(r.array().astype(np.float32), device).contiguous())
        elif marker == b'J':
            sd[name] = _to_device(r.array(), device).to(torch.int32)
        else:
            raise ValueError(f"{path}: unknown chunk marker {marker!r} for {name!r}")
    return sd, config


def _write_array(f, a: np.ndarray):
    a = np.ascontiguousarray(a)
    f.write(struct.pack('<BB', _CODES[a.dtype], a.ndim))
    for d in a.shape:
        f.write(struct.pack('<I', d))
    f.write(a.tobytes())


def _bitmask(codes: torch.Tensor):
    """(bitmask bytes, sign bytes, num_nonzero) of int8 codes, LSB first."""
    c = codes.reshape(-1).to(torch.int8).cpu().numpy()
    nz = c != 0
    return (np.packbits(nz, bitorder='little'), np.packbits(c[nz] == 1, bitorder='little'), int(nz.sum()))


def save_walsh(path: str, state_dict: dict, config: dict):
    """Write ``state_dict`` as a .walsh v4 file with the entry kinds of
    compress.py:189-348 (entries it does not cover, such as the mHC mappings,
    are skipped there and here).  Ternary weights are quantised with the
    absmean codes of walsh_ternary_quantize (the codes the layers compute
    with); float tensors are stored as float16, embeddings as int8 with a
    max-abs scale (compress.py:96-109)."""
    tok = state_dict.get('tok_embeddings.weight')
    out_w = state_dict.get('output.weight')
    tied = tok is not None and out_w is not None and tok.data_ptr() == out_w.data_ptr()
    with open(path, 'wb') as f:
        f.write(MAGIC)
        f.write(struct.pack('<H', VERSION))
        cfg = json.dumps(config).encode('utf-8')
        f.write(struct.pack('<I', len(cfg)))
        f.write(cfg)

        def head(marker, name):
            nb = name.encode('utf-8')
            f.write(marker + struct.pack('<H', len(nb)) + nb)

        for name, t in state_dict.items():
            t = t.detach()
            if name == 'tok_embeddings.weight' or (name == 'output.weight' and not tied):
                if name == 'output.weight' and tied:
                    continue
                mx = t.abs().max().item()
                scale = mx / 127.0 if mx > 0 else 1.0
                q = torch.round(t.float() / scale).clamp(-127, 127).to(torch.int8).cpu().numpy()
                head(b'E', name)
                f.write(struct.pack('<f', scale))
                _write_array(f, q)
            elif name.endswith('.weight') and any(k in name for k in _TERNARY_KEYS):
                codes = kernels.ternary_quantize(t.float().to('cuda' if not t.is_cuda else t.device),
                                                 codes=True, packed=False)['codes']
                bm, sg, nnz = _bitmask(codes)
                head(b'B', name)
                f.write(struct.pack('<B', t.dim()))
                for d in t.shape:
                    f.write(struct.pack('<I', d))
                f.write(struct.pack('<I', nnz))
                f.write(struct.pack('<I', len(bm)))
                f.write(bm.tobytes())
                f.write(struct.pack('<I', len(sg)))
                f.write(sg.tobytes())
            elif '.beta' in name and 'head_mixer' not in name:
                head(b'S', name)
                _write_array(f, t.float().cpu().numpy().astype(np.float16))
            elif '.alpha' in name:
                head(b'L', name)
                _write_array(f, t.float().cpu().numpy().astype(np.float16))
            elif 'norm' in name:
                head(b'N', name)
                _write_array(f, t.float().cpu().numpy().astype(np.float16))
            elif 'freqs_cis' in name:
                head(b'R', name)
                _write_array(f, torch.view_as_real(t).float().cpu().numpy())
            elif 'head_mixer.W' in name:
                head(b'H', name)
                _write_array(f, t.float().cpu().numpy().astype(np.float16))
            elif 'head_mixer.beta' in name:
                head(b'h', name)
                _write_array(f, t.float().cpu().numpy().astype(np.float16))
        f.write(b'END!')


__all__ = ["load_walsh", "save_walsh", "MAGIC", "VERSION"]
