"""taco_amd: an MI355X (gfx950) backend for HardShell, the integer GPT-2 engine of taco.

`taco_amd.hip` mirrors the hardshell-cuda API over the C ABI of libhardshell_hip.so
(include/hardshell_hip.h); `taco_amd.fold` is the host harness that plays taco's role above it
(windows, range coder, payloads, container)."""

__all__ = ["hip"]
