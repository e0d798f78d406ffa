"""Lowering of the scan and conv kinds (ssd, ssd_chunked, conv1d)."""

from __future__ import annotations

from . import abi


def lower_ssd(dp, spec):
    raise abi.HipBackendError("lower", abi.TH_ERR_UNSUPPORTED, "the SSD kernel is not built yet", spec.name)


def lower_conv1d(dp, spec):
    raise abi.HipBackendError("lower", abi.TH_ERR_UNSUPPORTED, "the conv1d kernel is not built yet", spec.name)
