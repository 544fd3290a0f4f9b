"""Engine constants and the frozen Settings (mirror of goi_jax/box2d/settings.py:17-107).

Every float is the float32 Box2D 2.3.1 holds, computed the way b2Settings.h computes it (left to right in float32),
so the GPU step and the reference start from bit-identical constants. Settings is a frozen dataclass of Python
scalars and numpy float32; `to_c()` packs it into the C ABI's GoiSettings (include/goi_b2.h).
"""
from dataclasses import dataclass, replace

import numpy as np

F32 = np.float32

# b2Settings.h v2.3.1 compile-time constants (settings.py:17-28)
PI = F32(3.14159265359)  # b2_pi
EPSILON = F32(np.finfo(np.float32).eps)  # b2_epsilon
MAX_FLOAT = F32(np.finfo(np.float32).max)  # b2_maxFloat
MAX_MANIFOLD_POINTS = 2
MAX_POLYGON_VERTICES = 8
AABB_EXTENSION = F32(0.1)
AABB_MULTIPLIER = F32(2.0)
MAX_SUB_STEPS = 8
MAX_TOI_CONTACTS = 32
MAX_CONDITION_NUMBER = F32(1000.0)
K_TOL = F32(0.1)


def deg2rad(deg):
    """Unity's value * Mathf.Deg2Rad in float32 (settings.py:31-33)."""
    return F32(F32(deg) * F32(0.0174532924))


def _stock_angle(deg):
    """b2Settings.h `(deg / 180.0f * b2_pi)` left to right in float32 (settings.py:36-38)."""
    return F32(F32(F32(deg) / F32(180.0)) * PI)


@dataclass(frozen=True)
class Settings:
    """World constants (b2Settings globals plus b2World flags); defaults are stock Box2D 2.3.1, Settings.game() is
    Getting Over It. Field names, defaults and meaning follow settings.py:42-80. `solver` picks the backend of
    `step`: "hip" (the MI355X kernels, default). `max_events` caps TOI events per step (None: the reference default
    C * (b2_maxSubSteps + 1) + 8, toi.py:838-840)."""
    gravity: tuple = (F32(0.0), F32(-10.0))
    velocity_iterations: int = 8
    position_iterations: int = 3
    linear_slop: F32 = F32(0.005)
    angular_slop: F32 = _stock_angle(2.0)
    polygon_radius: F32 = F32(F32(2.0) * F32(0.005))
    velocity_threshold: F32 = F32(1.0)
    max_linear_correction: F32 = F32(0.2)
    max_angular_correction: F32 = _stock_angle(8.0)
    max_translation: F32 = F32(2.0)
    max_rotation: F32 = F32(F32(0.5) * PI)
    baumgarte: F32 = F32(0.2)
    toi_baumgarte: F32 = F32(0.75)
    time_to_sleep: F32 = F32(0.5)
    linear_sleep_tolerance: F32 = F32(0.01)
    angular_sleep_tolerance: F32 = _stock_angle(2.0)
    clamps_per_second: bool = False
    allow_sleep: bool = True
    warm_starting: bool = True
    continuous_physics: bool = False
    unity_toi: bool = False
    toi_tie_oldest: bool = False
    auto_clear_forces: bool = True
    revolute_v24: bool = True
    solver: str = "hip"
    max_events: object = None

    @classmethod
    def stock(cls, **kw):
        return replace(cls(), **{k: _cast(v) for k, v in kw.items()})

    @classmethod
    def game(cls, **kw):
        """Getting Over It's Physics2D settings (settings.py:87-95)."""
        s = cls(gravity=(F32(0.0), F32(-30.0)), velocity_iterations=300, position_iterations=30,
                velocity_threshold=F32(1.0), max_linear_correction=F32(0.2), max_angular_correction=deg2rad(8),
                max_translation=F32(100.0), max_rotation=deg2rad(360), baumgarte=F32(0.4), toi_baumgarte=F32(0.75),
                time_to_sleep=F32(0.5), linear_sleep_tolerance=F32(0.01), angular_sleep_tolerance=deg2rad(2),
                linear_slop=F32(0.005), polygon_radius=F32(0.01), continuous_physics=True, unity_toi=True,
                toi_tie_oldest=True)
        return replace(s, **{k: _cast(v) for k, v in kw.items()})

    def to_c(self):
        """The C ABI struct (include/goi_b2.h GoiSettings)."""
        from ._abi import GoiSettings
        f = lambda n: float(F32(getattr(self, n)))  # noqa: E731
        return GoiSettings(
            velocity_iterations=int(self.velocity_iterations), position_iterations=int(self.position_iterations),
            linear_slop=f("linear_slop"), angular_slop=f("angular_slop"), polygon_radius=f("polygon_radius"),
            velocity_threshold=f("velocity_threshold"), max_linear_correction=f("max_linear_correction"),
            max_angular_correction=f("max_angular_correction"), max_translation=f("max_translation"),
            max_rotation=f("max_rotation"), baumgarte=f("baumgarte"), toi_baumgarte=f("toi_baumgarte"),
            time_to_sleep=f("time_to_sleep"), linear_sleep_tolerance=f("linear_sleep_tolerance"),
            angular_sleep_tolerance=f("angular_sleep_tolerance"), clamps_per_second=int(self.clamps_per_second),
            allow_sleep=int(self.allow_sleep), warm_starting=int(self.warm_starting),
            continuous_physics=int(self.continuous_physics), unity_toi=int(self.unity_toi),
            toi_tie_oldest=int(self.toi_tie_oldest), auto_clear_forces=int(self.auto_clear_forces),
            revolute_v24=int(self.revolute_v24), max_events=-1 if self.max_events is None else int(self.max_events))


def _cast(v):
    if v is None or isinstance(v, str):
        return v
    if isinstance(v, (bool, int, np.integer)) and not isinstance(v, (float, np.floating)):
        return v
    if isinstance(v, tuple):
        return tuple(F32(x) for x in v)
    return F32(v)
