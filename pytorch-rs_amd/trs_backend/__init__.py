"""ctypes binding of libtrs_hip.so (include/trs_hip.h) and libtrs_inputs.so.

This is the binding a Python caller of the C ABI uses; the torch_rs package
in this directory goes through the C++ host engine instead.
"""
from .abi import (  # noqa: F401
    Layout, TrsError, lib, inputs_lib, check, layout_of, contiguous_strides,
    DeviceArray, device_count, synchronize,
)
