"""The reference's module name (python/bindings.cpp:63): ``import vectorcore
as vc`` gives the same module surface as ``vectorcore_amd``, with the MI355X
``hip`` device next to ``cpu``, so the reference's examples and tests run
unchanged."""

from vectorcore_amd import *  # noqa: F401,F403
from vectorcore_amd import DEVICES, _vectorcore  # noqa: F401
