"""MI355X-native backend for the Big-LaMa generator forward pass.

`host_api` binds liblama_host.so (weights container, fixtures, PNG, window
geometry); `hip_engine` binds liblama_hip.so, the C-ABI engine that replaces
the reference's CUDA engine.
"""
from . import host_api, hip_engine  # noqa: F401

__all__ = ["host_api", "hip_engine", "PKG_DIR"]

import os as _os

PKG_DIR = _os.path.dirname(_os.path.abspath(__file__))
