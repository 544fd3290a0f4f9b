"""MI355X batched Box2D 2.3.1 world step: the drop-in for goi_jax.box2d (goi_jax/box2d/__init__.py:62-68).

    box2d = importlib.import_module("getting-over-it-rl_amd.box2d")
    d = box2d.WorldDef(box2d.Settings.stock(gravity=(0, -9.81), continuous_physics=True))
    ...; model, state = d.build(contact_capacity=40)
    model, state = box2d.prepare(model, state)                   # compact fixture layout
    dev = box2d.layout.to_device(box2d.world.batch(state, 16384))
    dev = box2d.step(model, dev, settings, dt)

Same public names as the reference: Settings, step, Model, State, WorldDef, the body/joint enums and GAME_DT. The
step runs hand-written HIP kernels for gfx950 (libgoi_b2.so through the C ABI in include/goi_b2.h).
"""
import numpy as np

from . import debug, io, layout, record, scenes, shapes, world
from .settings import Settings
from .step import (collide_, debug_shapes, last_launch, make_debug, prepare, sincos, step, step_, step_n_,
                   world_manifolds)
from .world import (DYNAMIC, KINEMATIC, PRISMATIC, REVOLUTE, STATIC, WELD, Model, State, WorldDef, compact_model,
                    compact_state, expand_state)

GAME_DT = np.float32(0.008333334)  # Time.fixedDeltaTime (float32 nearest 1/120)

__all__ = ["Settings", "step", "step_", "step_n_", "collide_", "debug_shapes", "last_launch", "make_debug", "prepare",
           "sincos", "world_manifolds",
           "Model", "State",
           "WorldDef", "GAME_DT", "STATIC", "KINEMATIC", "DYNAMIC", "REVOLUTE", "PRISMATIC", "WELD", "compact_model",
           "compact_state", "expand_state", "debug", "io", "layout", "record", "scenes", "shapes", "world"]
