"""nablatensor_amd — MI355X (gfx950) fused forward+adjoint Monte-Carlo tape replay.

A drop-in for NablaTensor's `rocm` AadEngine path:
  * nablatensor_amd._host   C++ host layer (recording, products, engine SPI,
                            MonteCarlo facade) under the reference's names;
  * nablatensor_amd.rocm    ctypes binding of the C ABI (include/nablatensor_rocm.h);
  * libnt_rocm.so           the engine: tape lowering, hipRTC for gfx950, launch.
Both native libraries are built in-tree by nablatensor_amd/build.py; importing
this package without them raises rather than falling back to anything else.
"""
from __future__ import annotations

from pathlib import Path

_PKG = Path(__file__).resolve().parent

try:
    from . import _host  # noqa: F401
except ImportError as exc:  # pragma: no cover - exercised only on an unbuilt tree
    raise ImportError(f"nablatensor_amd native host module is not built ({exc}); "
                      "run `python nablatensor_amd/build.py`") from exc

from ._host import (  # noqa: E402,F401
    AadEngines, AadOpEnum, AadOptions, AadRecorder, AadResult, AadTape, ADouble, CorrelatedNormals, EquityMarket,
    ExoticProducts, HestonMarket, HestonModel, MarketRecord, MonteCarlo, OptionTypeEnum, Products, RocmAadEngine,
    TimeGrid, UnsupportedOperationException, WorstOfBasket, modelEquity, modelHeston, modelRecord, record,
)
from . import rocm  # noqa: E402,F401

__all__ = [
    "AadEngines", "AadOpEnum", "AadOptions", "AadRecorder", "AadResult", "AadTape", "ADouble", "CorrelatedNormals",
    "EquityMarket", "ExoticProducts", "HestonMarket", "HestonModel", "MarketRecord", "MonteCarlo", "OptionTypeEnum",
    "Products", "RocmAadEngine", "TimeGrid", "UnsupportedOperationException", "WorstOfBasket", "modelEquity",
    "modelHeston", "modelRecord", "record", "rocm",
]
