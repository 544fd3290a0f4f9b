"""Batches of States on the GPU in the kernels' worlds-minor layout, and back.

A device State has the reference's field names and logical shapes (N, *inner) (goi_jax/box2d/world.py:70-174), as
torch tensors whose storage is worlds-minor: leaf L with inner shape S is one contiguous (prod(S), pitch) buffer
viewed as (N, *S) with stride 1 on the world axis. `state_view` hands those buffers to the C ABI without copies.
"""
import numpy as np
import torch

from . import world as wd
from ._abi import GoiStateView

_TORCH = {np.dtype(np.float32): torch.float32, np.dtype(np.int32): torch.int32, np.dtype(bool): torch.bool}


def _dtype(dt):
    return _TORCH[np.dtype(dt)]


def packed_words(dims):
    """The packed layout of capacities dims = (B, R, J, C): words[l] = 4-byte words per unit of pitch before leaf l
    (each leaf's per-world bytes rounded up to a multiple of 4), words[-1] the whole; the library's goi_packed_layout
    gives the same table."""
    words = [0]
    for _, _, dt, inner in wd.LEAVES:
        nbytes = int(np.prod(wd.leaf_shape(inner, dims), dtype=np.int64)) * np.dtype(dt).itemsize
        words.append(words[-1] + (nbytes + 3) // 4)
    return words


def empty_device_state(n, dims, device="cuda", pitch=None, packed=True):
    """An uninitialised device State of n worlds with capacities dims = (B, R, J, C), pitch n by default. With a pitch
    that is a multiple of 64 the leaves are by default the consecutive parts of one buffer (the packed layout), which
    lets the step address every leaf from one base pointer; packed=False, or another pitch, gives one buffer per
    leaf."""
    pitch = n if pitch is None else pitch
    vals = []
    if packed and pitch > 0 and pitch % 64 == 0:
        words = packed_words(dims)
        buf = torch.empty(words[-1] * 4 * pitch, dtype=torch.uint8, device=device)
        for (_, _, dt, inner), w in zip(wd.LEAVES, words):
            shape = wd.leaf_shape(inner, dims)
            nbytes = int(np.prod(shape, dtype=np.int64)) * np.dtype(dt).itemsize * pitch
            part = buf[4 * w * pitch:4 * w * pitch + nbytes].view(_dtype(dt)).view(tuple(shape) + (pitch,))
            vals.append(part[..., :n].movedim(-1, 0))
        return wd.from_leaves(vals)
    for _, _, dt, inner in wd.LEAVES:
        shape = wd.leaf_shape(inner, dims)
        buf = torch.empty(tuple(shape) + (pitch,), dtype=_dtype(dt), device=device)
        vals.append(buf[..., :n].movedim(-1, 0))
    return wd.from_leaves(vals)


def to_device(state, device="cuda", pitch=None, packed=True):
    """A batched numpy State (leading world axis) to a device State (packed by default, as empty_device_state)."""
    leaves = wd.leaves(state)
    n = np.asarray(leaves[0]).shape[0]
    dims = wd.dims(state)
    out = empty_device_state(n, dims, device, pitch, packed)
    for dst, src in zip(wd.leaves(out), leaves):
        src = np.asarray(src)
        dst.copy_(torch.from_numpy(np.ascontiguousarray(src)).to(device))
    return out


def to_host(state):
    """A device State to a batched numpy State (contiguous, batch-major)."""
    return wd.from_leaves([np.ascontiguousarray(t.detach().cpu().numpy()) for t in wd.leaves(state)])


def clone(state):
    """A deep copy of a device State in the same layout."""
    leaves = wd.leaves(state)
    n = leaves[0].shape[0]
    dims = wd.dims(state)
    out = empty_device_state(n, dims, leaves[0].device)
    for dst, src in zip(wd.leaves(out), leaves):
        dst.copy_(src)
    return out


def pitch_of(state):
    """The worlds-minor pitch of a device State's leaves."""
    t = state.bodies.xf_p
    return t.stride(-1) if t.dim() > 1 else t.shape[0]


def state_view(state):
    """GoiStateView over a device State; checks the worlds-minor layout."""
    leaves = wd.leaves(state)
    n = leaves[0].shape[0]
    B, R, J, C = wd.dims(state)
    v = GoiStateView()
    v.n_worlds = n
    pitch = None
    device = None
    for t, (_, name, dt, inner) in zip(leaves, wd.LEAVES):
        if not isinstance(t, torch.Tensor) or not t.is_cuda:
            raise ValueError(f"leaf {name}: not a GPU tensor (move the State with layout.to_device)")
        if device is not None and t.device != device:
            raise ValueError(f"leaf {name}: on {t.device}, other leaves on {device}")
        device = t.device
        if t.dtype != _dtype(dt):
            raise TypeError(f"leaf {name}: dtype {t.dtype}, expected {_dtype(dt)}")
        shape = (n,) + wd.leaf_shape(inner, (B, R, J, C))
        if tuple(t.shape) != shape:
            raise ValueError(f"leaf {name}: shape {tuple(t.shape)}, expected {shape}")
        if t.dim() > 1:
            p = t.stride(-1)
            want, acc = [1], p
            for d in reversed(shape[1:]):
                want.insert(1, acc)
                acc *= d
            if tuple(t.stride()) != tuple(want) or p < n or (pitch is not None and p != pitch):
                raise ValueError(f"leaf {name}: not in the worlds-minor layout (strides {t.stride()})")
            pitch = p
        elif t.stride(0) != 1:
            raise ValueError(f"leaf {name}: world stride must be 1")
    v.pitch = n if pitch is None else pitch
    v.B, v.C, v.R, v.J = B, C, R, J
    for i, t in enumerate(leaves):
        v.leaf[i] = t.data_ptr()
    return v
