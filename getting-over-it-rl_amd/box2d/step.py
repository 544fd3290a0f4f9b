"""b2World::Step over a batch of worlds on the MI355X: the drop-in for goi_jax/box2d/step.py:28-47.

    model, state = WorldDef(settings) ... .build(contact_capacity=32)
    model = compact_model(model, state)                  # shared static terrain, as the reference GPU path needs
    dev = layout.to_device(world.batch(compact_state(model, state), 16384))
    dev = step(model, dev, settings, dt)                 # a new State (step_ steps in place)

`step(model, state, settings, dt, axis_name=None)` keeps the reference signature; axis_name is accepted and ignored
(the device kernels need no shared trip count, cf. goi_jax/box2d/gpu/solve.py:28). Settings.solver must be "hip":
there is no CPU fallback, a missing or unloadable libgoi_b2.so raises.
"""
import ctypes

import numpy as np
import torch

from . import _abi
from . import layout
from . import world as wd

_MODELS = {}


class DeviceModel:
    """The library's model handle (goi_model_create) for one compact Model, contact capacity and device."""

    def __init__(self, model, contact_capacity, device=None):
        self.L = _abi.lib()
        desc, self._keep = _abi.model_desc(model)
        handle = ctypes.c_void_p()
        dev = torch.device("cuda") if device is None else torch.device(device)
        with torch.cuda.device(dev):
            stream = torch.cuda.current_stream().cuda_stream
            _abi.check(self.L.goi_model_create(ctypes.byref(desc), int(contact_capacity), ctypes.c_void_p(stream),
                                               ctypes.byref(handle)), self.L)
        self.handle = handle
        self.device = dev
        self.capacity = int(contact_capacity)

    def __del__(self):
        if getattr(self, "handle", None) is not None and self.handle.value:
            try:
                self.L.goi_model_destroy(self.handle)
            except Exception:  # interpreter shutdown
                pass
            self.handle = None


def _compact_from_device_state(model, state):
    """compact_model (world.py:437-472) of a full-layout Model from a device State's fixture rows: the body types and
    the static fixtures' fat AABBs, friction and restitution must be the same in every world (checked on the device;
    a step never changes them), and world 0's become the Model's shared tables."""
    types = state.bodies.type
    if bool((types != types[:1]).any()):
        raise ValueError("compact_model: the worlds' body types differ, so static fixtures cannot be shared")
    types0 = types[:1].cpu().numpy()
    on_static = types0[0][np.asarray(model.fixture_body)] == wd.STATIC
    fx = state.fixtures
    if fx.fat.shape[1] != on_static.size:
        raise ValueError("a full-layout Model needs a full-layout State (a row per fixture)")
    idx = torch.as_tensor(np.flatnonzero(on_static), device=fx.fat.device, dtype=torch.long)
    for name, leaf in (("fat", fx.fat), ("friction", fx.friction), ("restitution", fx.restitution)):
        rows = leaf.index_select(1, idx)
        if bool((rows != rows[:1]).any()):
            raise ValueError(f"compact_model: a static fixture's {name} differs between worlds")
    host = wd.State(bodies=wd.Bodies(*[types0 if f == "type" else None for f in wd.Bodies._fields]),
                    fixtures=wd.Fixtures(friction=fx.friction[:1].cpu().numpy(),
                                         restitution=fx.restitution[:1].cpu().numpy(), fat=fx.fat[:1].cpu().numpy()),
                    joints=None, contacts=None, gravity=None, inv_dt0=None, next_key=None, new_fixture=None,
                    overflow=None)
    return wd.compact_model(model, host)


def device_model(model, contact_capacity, device=None, state=None):
    """Cached DeviceModel for (model object, capacity, device). A compact Model built without body types (the
    reference's compact_model keeps them in the State only, world.py:437-472) takes them from `state`, whose worlds
    must agree. A full-layout Model (WorldDef.build's) is compacted first from `state`'s static fixture rows, as the
    reference's GPU path does (gpu/pairs.py:286-303 read a compact Model's shared tables): its States may stay in the
    full layout, whose static rows the step leaves untouched."""
    key = (id(model), int(contact_capacity), str(device))
    hit = _MODELS.get(key)
    if hit is not None and hit[0] is model:
        return hit[1]
    desc_model = model
    if model.fixture_slot is None:
        if state is None:
            raise ValueError("a full-layout Model needs the State its static fixture rows come from")
        desc_model = _compact_from_device_state(model, state)
    elif model.body_type is None and state is not None:
        bt = np.asarray(state.bodies.type.to("cpu") if torch.is_tensor(state.bodies.type) else state.bodies.type)
        bt = bt.reshape(-1, bt.shape[-1])
        if not (bt == bt[0]).all():
            raise ValueError("the device step needs body types shared by every world (compact layout)")
        desc_model = model._replace(body_type=bt[0].astype(np.int32))
    dm = DeviceModel(desc_model, contact_capacity, device)
    _MODELS[key] = (model, dm)
    return dm


def step_(model, state, settings, dt, debug=None, stream=None):
    """One step of every world of a device State, in place. Returns the same State."""
    if getattr(settings, "solver", "hip") != "hip":
        raise ValueError(f"Settings.solver={settings.solver!r}: this package steps on the GPU only ('hip')")
    view = layout.state_view(state)
    C = state.contacts.pair.shape[-1]
    dev = state.contacts.pair.device
    dm = device_model(model, C, dev, state)
    cs = settings.to_c()
    st = torch.cuda.current_stream(dev).cuda_stream if stream is None else stream
    dbg = None if debug is None else ctypes.byref(debug)
    _abi.check(dm.L.goi_step(dm.handle, ctypes.byref(view), ctypes.byref(cs), ctypes.c_float(np.float32(dt)),
                             ctypes.c_void_p(st), dbg), dm.L)
    return state


def step_n_(model, state, settings, dt, n, debug=None, stream=None):
    """n consecutive steps of every world of a device State in one launch, in place: the same State as n calls of
    step_ with the joint motor commands and forces left as they are (a caller's physics sub-steps per action).
    Returns the same State."""
    if getattr(settings, "solver", "hip") != "hip":
        raise ValueError(f"Settings.solver={settings.solver!r}: this package steps on the GPU only ('hip')")
    view = layout.state_view(state)
    C = state.contacts.pair.shape[-1]
    dev = state.contacts.pair.device
    dm = device_model(model, C, dev, state)
    cs = settings.to_c()
    st = torch.cuda.current_stream(dev).cuda_stream if stream is None else stream
    dbg = None if debug is None else ctypes.byref(debug)
    _abi.check(dm.L.goi_step_n(dm.handle, ctypes.byref(view), ctypes.byref(cs), ctypes.c_float(np.float32(dt)),
                               ctypes.c_int32(int(n)), ctypes.c_void_p(st), dbg), dm.L)
    return state


def step(model, state, settings, dt, axis_name=None):
    """b2World::Step (step.py:28-47) of a batched device State; returns a new State (the input is unchanged)."""
    del axis_name
    out = layout.clone(state)
    return step_(model, out, settings, dt)


def collide_(model, state, settings, stream=None):
    """Broadphase + narrowphase only, in place: start-of-step FindNewContacts where new_fixture, then Collide."""
    view = layout.state_view(state)
    C = state.contacts.pair.shape[-1]
    dev = state.contacts.pair.device
    dm = device_model(model, C, dev, state)
    cs = settings.to_c()
    st = torch.cuda.current_stream(dev).cuda_stream if stream is None else stream
    _abi.check(dm.L.goi_collide(dm.handle, ctypes.byref(view), ctypes.byref(cs), ctypes.c_void_p(st)), dm.L)
    return state


def world_manifolds(model, state, stream=None):
    """b2WorldManifold of every contact slot of a device State: (normal (N, C, 2), points (N, C, 2, 2),
    separations (N, C, 2)) float32 CUDA tensors (worlds-minor storage); zeros where a slot is free or has no point."""
    view = layout.state_view(state)
    n, C = state.contacts.pair.shape
    dev = state.contacts.pair.device
    dm = device_model(model, C, dev, state)
    pitch = view.pitch
    bufs = [torch.zeros(shape + (pitch,), dtype=torch.float32, device=dev) for shape in ((C, 2), (C, 2, 2), (C, 2))]
    st = torch.cuda.current_stream(dev).cuda_stream if stream is None else stream
    _abi.check(dm.L.goi_world_manifold(dm.handle, ctypes.byref(view), *[ctypes.c_void_p(b.data_ptr()) for b in bufs],
                                       ctypes.c_void_p(st)), dm.L)
    return tuple(b[..., :n].movedim(-1, 0) for b in bufs)


def last_launch():
    """The calling thread's last step or collide launch (goi_last_launch): dict(worlds_per_wave, blocks, lds_bytes,
    kernel), kernel one of "generic", "rig", "island", "collide"."""
    L = _abi.lib()
    info = _abi.GoiLaunchInfo()
    _abi.check(L.goi_last_launch(ctypes.byref(info)), L)
    names = {_abi.KERNEL_GENERIC: "generic", _abi.KERNEL_RIG: "rig", _abi.KERNEL_ISLAND: "island",
             _abi.KERNEL_COLLIDE: "collide"}
    return dict(worlds_per_wave=info.worlds_per_wave, blocks=info.blocks, lds_bytes=info.lds_bytes,
                kernel=names.get(info.kernel))


def sincos(x):
    """(float)sin((double)x), (float)cos((double)x) of a float32 CUDA tensor, as the kernels compute them."""
    L = _abi.lib()
    x = x.contiguous()
    s, c = torch.empty_like(x), torch.empty_like(x)
    st = torch.cuda.current_stream(x.device).cuda_stream
    _abi.check(L.goi_sincos(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(s.data_ptr()),
                            ctypes.c_void_p(c.data_ptr()), ctypes.c_int32(x.numel()), ctypes.c_void_p(st)), L)
    return s, c


def debug_shapes(n, dims):
    """{GoiDebug field: (rows, n)} of the debug arrays for n worlds (or a pitch of n) of capacities dims = (B, R, J,
    C)."""
    B, _, _, C = dims
    E, Rw = _abi.DEBUG_TOI_EVENTS, _abi.DEBUG_TOI_ROWS
    return dict(body_island=(B, n), contact_island=(C, n), contact_order=(C, n), n_islands=(n,),
                toi_event_slot=(E, n), toi_event_alpha=(E, n), toi_event_island=(E, n), toi_island_rows=(E * Rw, n),
                status=(n,))


def make_debug(n, dims, device="cuda", pitch=None):
    """GoiDebug buffers (islands, solve order, TOI event traces) for a device State of n worlds whose leaves have the
    given pitch (n by default; the kernels write element (i, w) at [i * pitch + w]); returns (struct, tensors) with
    the tensors as (rows, pitch)."""
    t = {k: torch.full(shape, -7, dtype=torch.int32, device=device)
         for k, shape in debug_shapes(n if pitch is None else pitch, dims).items()}
    d = _abi.GoiDebug()
    for k, v in t.items():
        setattr(d, k, ctypes.c_void_p(v.data_ptr()))
    return d, t


def prepare(model, state):
    """(compact Model, compact State) from a WorldDef build, as the device step expects."""
    cm = wd.compact_model(model, state)
    return cm, wd.compact_state(cm, state)
