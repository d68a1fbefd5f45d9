"""ORACLE -- test infrastructure only.

numpy restatement of the weight-sync byte movement:

  expand_entries   the strided push-entry expansion of
                   WeightSynchronizerBase::PushWeightsResharded
                   (tpu_sync/weight_sync/weight_synchronizer_base.cc:626-666):
                   count <= 0 means 1; count == 1 or a contiguous entry
                   (src_stride == dst_stride == size) is one task of
                   count * size bytes, otherwise one task per row c at
                   src_offset + c * src_stride -> dst_offset + c * dst_stride.
  apply_entries    performs those tasks between two byte buffers.
  nd_shard_slices  compute_nd_shard_slices (tpu_sync/kv_cache/
                   nd_slice_math.py:23-70): tile = extent // mesh, the last
                   shard of each dimension takes the remainder, shards in
                   row-major order.
  offset_table     the packed host layout of this build: tensors in order,
                   each starting at a multiple of 256 bytes.

Parity status: expand_entries / nd_shard_slices are pinned by known answers
derived from the definitions and by closed forms (a column split equals
numpy column slicing; pack then unpack is the identity). offset_table /
pack have no reference counterpart (the reference keeps one host buffer per
tensor): the packed host layout is this build's own format, so its
definition is what fixes it, and it is pinned by known answers derived from
that definition (offsets of hand-picked tensor sizes) and by the byte
identity of every tensor's copy.
"""
import itertools

import numpy as np


def expand_entries(entries):
    """entries: iterables (src_off, dst_off, size, count, src_stride, dst_stride)
    -> list of (src_off, dst_off, nbytes) tasks."""
    tasks = []
    for src_off, dst_off, size, count, src_stride, dst_stride in entries:
        count = count if count > 0 else 1
        if count == 1 or (src_stride == size and dst_stride == size):
            tasks.append((src_off, dst_off, count * size))
        else:
            for c in range(count):
                tasks.append((src_off + c * src_stride, dst_off + c * dst_stride, size))
    return tasks


def apply_entries(src, dst, entries):
    """Copies per expand_entries between uint8 arrays (offsets are into them)."""
    for s, d, n in expand_entries(entries):
        dst[d:d + n] = src[s:s + n]
    return dst


def nd_shard_slices(global_shape, mesh_shape):
    if len(global_shape) != len(mesh_shape):
        raise ValueError("rank mismatch")
    tiles = [g // m for g, m in zip(global_shape, mesh_shape)]
    out = []
    for coord in itertools.product(*[range(m) for m in mesh_shape]):
        out.append([(c * tiles[d], (c + 1) * tiles[d] if c < mesh_shape[d] - 1
                     else global_shape[d]) for d, c in enumerate(coord)])
    return out


def offset_table(sizes, align=256):
    offs, pos = [], 0
    for n in sizes:
        offs.append(pos)
        pos = (pos + n + align - 1) // align * align
    return offs, pos


def pack(tensors_u8, align=256):
    """Packed image of uint8 arrays per offset_table (padding zero)."""
    offs, total = offset_table([t.size for t in tensors_u8], align)
    img = np.zeros(total, np.uint8)
    for t, o in zip(tensors_u8, offs):
        img[o:o + t.size] = t
    return img, offs
