"""Model and State interchange: .npz files and DLPack.

Files hold the reference's pytree layout (goi_jax/box2d/world.py:30-174): one array per leaf, batch-major
(N, *inner), keyed "<group>.<field>" ("bodies.c", "contacts.pair", "gravity", ...), and are read without pickling
(numpy.load with allow_pickle=False). DLPack moves leaves between this package's device States (worlds-minor
storage) and any array library that speaks the protocol (JAX, PyTorch, CuPy) in the reference's batch-major layout.
"""
import numpy as np

from . import world as wd

_MODEL_OPTIONAL = {f for f in wd.Model._fields if wd.Model._field_defaults.get(f, 0) is None}


def _key(group, name):
    return name if group is None else f"{group}.{name}"


def save_state(path, state):
    """Write a State (numpy, or a device State of torch tensors) to an .npz file, batch-major."""
    vals = [np.asarray(x.detach().cpu().numpy()) if hasattr(x, "detach") else np.asarray(x) for x in wd.leaves(state)]
    np.savez(path, **{_key(g, n): v for (g, n, _, _), v in zip(wd.LEAVES, vals)})


def load_state(path):
    """A numpy State from an .npz file written by save_state; checks every leaf's dtype and its shape against the
    capacities the file implies."""
    with np.load(path, allow_pickle=False) as f:
        missing = [_key(g, n) for g, n, _, _ in wd.LEAVES if _key(g, n) not in f.files]
        if missing:
            raise ValueError(f"{path}: missing leaves {missing[:4]}")
        vals = [f[_key(g, n)] for g, n, _, _ in wd.LEAVES]
    st = wd.from_leaves(vals)
    dims = wd.dims(st)
    lead = vals[0].shape[:vals[0].ndim - len(wd.leaf_shape(wd.LEAVES[0][3], dims))]
    for (g, n, dt, inner), v in zip(wd.LEAVES, vals):
        if v.dtype != np.dtype(dt):
            raise TypeError(f"{path}: leaf {_key(g, n)} has dtype {v.dtype}, expected {np.dtype(dt)}")
        if v.shape != tuple(lead) + wd.leaf_shape(inner, dims):
            raise ValueError(f"{path}: leaf {_key(g, n)} has shape {v.shape}")
    return st


def save_model(path, model):
    """Write a Model to an .npz file (fields that are None are left out)."""
    np.savez(path, **{k: np.asarray(v) for k, v in model._asdict().items() if v is not None})


def load_model(path):
    """A Model from an .npz file written by save_model."""
    with np.load(path, allow_pickle=False) as f:
        fields = {k: f[k] for k in f.files}
    unknown = set(fields) - set(wd.Model._fields)
    if unknown:
        raise ValueError(f"{path}: unknown Model fields {sorted(unknown)}")
    required = [k for k in wd.Model._fields if k not in _MODEL_OPTIONAL]
    missing = [k for k in required if k not in fields]
    if missing:
        raise ValueError(f"{path}: missing Model fields {missing}")
    return wd.Model(**fields)


def from_dlpack(state, device="cuda", pitch=None):
    """A device State from a State whose leaves speak DLPack (JAX arrays, torch tensors, ...) in the reference's
    batch-major layout (N, *inner): each leaf is taken without a copy where the producer allows and copied once into
    the worlds-minor storage the kernels use."""
    import torch

    from . import layout
    leaves = [torch.from_dlpack(x) for x in wd.leaves(state)]
    n = leaves[0].shape[0]
    dims = wd.dims(wd.from_leaves(leaves))
    out = layout.empty_device_state(n, dims, device, pitch)
    for dst, src, (g, name, dt, _) in zip(wd.leaves(out), leaves, wd.LEAVES):
        if src.dtype != dst.dtype:
            raise TypeError(f"leaf {_key(g, name)}: dtype {src.dtype}, expected {dst.dtype}")
        if tuple(src.shape) != tuple(dst.shape):
            raise ValueError(f"leaf {_key(g, name)}: shape {tuple(src.shape)}, expected {tuple(dst.shape)}")
        dst.copy_(src)
    return out


def to_dlpack(state):
    """A State of contiguous batch-major torch tensors (copies of a device State's leaves, on its device), each
    of which any DLPack consumer can take (jax.dlpack.from_dlpack, numpy.from_dlpack for host tensors)."""
    return wd.from_leaves([x.contiguous() for x in wd.leaves(state)])
