"""mojoboost-amd: the mojotrees GBDT training path on AMD Instinct MI355X.

Estimators (`MojoTreesRegressor`, `MojoTreesClassifier`) and the device-level
API (`device.Dataset`) call the HIP library libmojoboost_hip.so through
ctypes; see include/mojotrees.h and include/mojoboost_hip.h.
"""
from .sklearn import MojoTreesClassifier, MojoTreesRegressor  # noqa: F401

__version__ = "0.1.0"
