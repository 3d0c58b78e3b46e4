"""XFA1 flash-attention captures: read, write and replay through the library.

The capture format is the one the reference writes for its first multi-query
FLASH_ATTN_EXT node (src/bridge/session.cpp:493-533, fa-probe.bin):

    uint32 magic 0x31414658 ("XFA1"), uint32 count (5: q, k, v, mask, output)
    per tensor: int32 index, int32 op, int32 type,
                int64 ne[4], uint64 nb[4], uint64 bytes, char name[64],
                bytes of raw data (the tensor's span from its data pointer)

``bytes`` is ggml_nbytes of the node, the extent its strides reach:
``type_size + sum((ne[i] - 1) * nb[i])`` for one-element blocks and
``ne[0] * nb[0] / block + sum_{i>0}((ne[i] - 1) * nb[i])`` for block types.
The op parameters (scale, max_bias, logit_softcap) and attention sinks are not
part of the capture, so a replay takes the parameters as arguments (the default
scale is 1/sqrt(head dim)) and runs without sinks. A capture whose writer
failed part way (the reference logs "fa-probe: FAILED") is truncated and the
reader rejects it.

``python -m xqattn.xfa1 fa-probe.bin [--scale S]`` replays a capture on the GPU
and prints the largest difference from the captured output.
"""
from __future__ import annotations

import argparse
import dataclasses
import math
import struct
import sys

import numpy as np

from .workloads import BLOCK, F32, TYPE_SIZE, HostTensor

MAGIC = 0x31414658
ROLES = ("q", "k", "v", "mask", "output")
_HEAD = struct.Struct("<3i4q4QQ64s")


@dataclasses.dataclass
class CapturedTensor:
    index: int
    op: int
    type: int
    ne: tuple
    nb: tuple
    name: str
    raw: np.ndarray  # uint8 span

    def host(self) -> HostTensor:
        return HostTensor(self.type, tuple(self.ne), tuple(self.nb), self.raw)


def span_bytes(typ: int, ne, nb) -> int:
    """The byte extent of a tensor view (ggml_nbytes)."""
    if min(ne) <= 0:
        return 0
    if BLOCK[typ] == 1:
        return TYPE_SIZE[typ] + sum((ne[i] - 1) * nb[i] for i in range(4))
    return ne[0] * nb[0] // BLOCK[typ] + sum((ne[i] - 1) * nb[i] for i in range(1, 4))


def read(path) -> dict:
    """-> {"q": CapturedTensor, "k": ..., "v": ..., "mask": ..., "output": ...}"""
    data = open(path, "rb").read()
    if len(data) < 8:
        raise ValueError("XFA1: truncated header")
    magic, count = struct.unpack_from("<2I", data, 0)
    if magic != MAGIC:
        raise ValueError(f"XFA1: bad magic {magic:#x}")
    if count != len(ROLES):
        raise ValueError(f"XFA1: {count} tensors, expected {len(ROLES)}")
    off = 8
    out = {}
    for role in ROLES:
        if off + _HEAD.size > len(data):
            raise ValueError(f"XFA1: truncated record for {role}")
        f = _HEAD.unpack_from(data, off)
        off += _HEAD.size
        index, op, typ = f[0], f[1], f[2]
        ne, nb, nbytes, name = tuple(f[3:7]), tuple(f[7:11]), f[11], f[12]
        if index != ROLES.index(role):
            raise ValueError(f"XFA1: record {index} where {ROLES.index(role)} ({role}) was expected")
        if typ not in TYPE_SIZE:
            raise ValueError(f"XFA1: {role} has unsupported type {typ}")
        if nbytes != span_bytes(typ, ne, nb):
            raise ValueError(f"XFA1: {role} holds {nbytes} bytes, its view spans {span_bytes(typ, ne, nb)}")
        if off + nbytes > len(data):
            raise ValueError(f"XFA1: truncated data for {role}")
        raw = np.frombuffer(data, np.uint8, nbytes, off).copy()
        off += nbytes
        out[role] = CapturedTensor(index, op, typ, ne, nb, name.split(b"\0", 1)[0].decode(errors="replace"), raw)
    if off != len(data):
        raise ValueError(f"XFA1: {len(data) - off} trailing bytes")
    return out


def write(path, tensors: dict, ops: dict | None = None, names: dict | None = None) -> None:
    """Write host tensors {role: HostTensor} in the capture's layout (the mask
    may be None only if the caller accepts a capture the reader rejects)."""
    ops = ops or {}
    names = names or {}
    with open(path, "wb") as fp:
        fp.write(struct.pack("<2I", MAGIC, len(ROLES)))
        for i, role in enumerate(ROLES):
            t = tensors[role]
            nbytes = span_bytes(t.type, t.ne, t.nb)
            raw = np.ascontiguousarray(t.buf).reshape(-1).view(np.uint8)[:nbytes]
            if raw.size != nbytes:
                raise ValueError(f"{role}: buffer holds {raw.size} bytes, its view spans {nbytes}")
            name = names.get(role, role).encode()[:63]
            fp.write(_HEAD.pack(i, ops.get(role, 0), t.type, *t.ne, *t.nb, nbytes, name))
            fp.write(raw.tobytes())


def replay(path, scale: float | None = None, max_bias: float = 0.0, softcap: float = 0.0,
           qk_policy: int | None = None, split_mode: int | None = None, engine: int | None = None):
    """Run a capture's q, k, v, mask through xq_flash_attn_ext on the GPU, into
    an output of the captured output's type, shape and strides.
    Returns (got, want): float32 arrays in ne order [ne3][ne2][ne1][ne0]."""
    import torch

    from . import ENGINE_AUTO, QK_CONSISTENT, SPLIT_AUTO, DevTensor, fa_params, flash_attn_ext

    cap = read(path)
    q, k, v, m, o = (cap[r].host() for r in ROLES)
    if o.type != F32:
        raise ValueError("XFA1 replay: the captured output must be F32")
    scale = 1.0 / math.sqrt(q.ne[0]) if scale is None else scale
    dq, dk, dv, dm = (DevTensor.from_host(t) for t in (q, k, v, m))
    dd = DevTensor.empty_like_host(HostTensor(o.type, o.ne, o.nb, np.zeros(o.buf.size, np.uint8)))
    p = fa_params(scale, max_bias, softcap, QK_CONSISTENT if qk_policy is None else qk_policy,
                  SPLIT_AUTO if split_mode is None else split_mode, ENGINE_AUTO if engine is None else engine)
    flash_attn_ext(dq, dk, dv, dm, None, dd, p)
    torch.cuda.synchronize()
    got = gather_f32(HostTensor(o.type, o.ne, o.nb, dd.to_host_bytes()))
    return got, gather_f32(o)


def gather_f32(t: HostTensor) -> np.ndarray:
    """The f32 elements of a (possibly strided) view, in ne order [ne3][ne2][ne1][ne0]."""
    if t.type != F32:
        raise ValueError("gather_f32: not an F32 tensor")
    ne, nb = t.ne, t.nb
    if min(ne) <= 0:
        return np.zeros(tuple(reversed(ne)), np.float32)
    base = np.ascontiguousarray(t.buf).reshape(-1).view(np.uint8)
    off = (np.arange(ne[3])[:, None, None, None] * nb[3] + np.arange(ne[2])[None, :, None, None] * nb[2] +
           np.arange(ne[1])[None, None, :, None] * nb[1] + np.arange(ne[0])[None, None, None, :] * nb[0])
    words = base[off.reshape(-1)[:, None] + np.arange(4)]
    return np.ascontiguousarray(words).view(np.float32).reshape(ne[3], ne[2], ne[1], ne[0])


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="replay an XFA1 flash-attention capture on the GPU")
    ap.add_argument("capture")
    ap.add_argument("--scale", type=float, default=None, help="kq scale (default 1/sqrt(head dim))")
    ap.add_argument("--max-bias", type=float, default=0.0)
    ap.add_argument("--softcap", type=float, default=0.0)
    args = ap.parse_args(argv)
    got, want = replay(args.capture, args.scale, args.max_bias, args.softcap)
    err = np.abs(got.astype(np.float64) - want)
    print(f"{args.capture}: shape {got.shape}, max |gpu - captured| = {np.nanmax(err):.3e}, "
          f"max |captured| = {np.nanmax(np.abs(want)):.3e}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
