"""getting-over-it-rl_amd: the MI355X-native batched Box2D 2.3.1 world step of miwate/getting-over-it-rl.

The package name is not a Python identifier; load it with importlib:

    goi = importlib.import_module("getting-over-it-rl_amd")
    box2d = goi.box2d
"""
from . import box2d  # noqa: F401
