"""HephaestusError vocabulary (crates/hephaestus-core/src/domain/error.rs:8-58).

Each C-ABI status code maps to one subclass; the display strings follow the
reference's `#[error(...)]` attributes, and `.message` carries the backend
detail exactly as the library reported it.
"""
from __future__ import annotations


class HephaestusError(Exception):
    """Base of every error raised by this package."""

    prefix = ""

    def __init__(self, message: str = ""):
        self.message = message
        super().__init__(f"{self.prefix}{message}")


class AdapterUnavailable(HephaestusError):
    prefix = "no compatible accelerator adapter available: "


class DeviceUnavailable(HephaestusError):
    prefix = "accelerator device creation failed: "


class AllocationFailed(HephaestusError):
    prefix = "accelerator allocation failed: "


class DispatchFailed(HephaestusError):
    prefix = "kernel dispatch failed: "


class InvalidConfiguration(HephaestusError):
    prefix = "invalid configuration: "


class TransferFailed(HephaestusError):
    prefix = "device transfer failed: "


class LengthMismatch(HephaestusError):
    """error.rs:30-36: carries the two element counts."""

    def __init__(self, host_len: int, device_len: int):
        self.host_len = host_len
        self.device_len = device_len
        msg = f"host length {host_len} does not match device buffer length {device_len}"
        self.message = msg
        Exception.__init__(self, msg)


BY_STATUS = {
    1: AdapterUnavailable,
    2: DeviceUnavailable,
    3: AllocationFailed,
    5: DispatchFailed,
    6: InvalidConfiguration,
    7: TransferFailed,
}
