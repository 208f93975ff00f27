"""Shared test helpers (re-exported from oracle/device_io.py)."""

from oracle.device_io import *  # noqa: F401,F403
from oracle.device_io import (bank_from_dev, bank_to_dev, cosine, dev_bf16, dev_i32,  # noqa: F401
                              host_bf16, host_u32, layer_from_dev, layer_to_dev)
