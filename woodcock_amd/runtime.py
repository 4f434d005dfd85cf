"""Per-device runtime plumbing: workspaces, device ints, the stream handle.

PyTorch-ROCm provides device memory and streams; every computation goes
through libwoodcock_hip.so.
"""
from __future__ import annotations

import ctypes as C

import torch

from . import _lib

_workspaces: dict[tuple[int, int], torch.Tensor] = {}


def device_of(t: torch.Tensor) -> torch.device:
    if t.device.type != "cuda":
        raise ValueError(f"expected a GPU tensor, got a tensor on {t.device}")
    return t.device


def stream_ptr(stream: torch.cuda.Stream | None = None):
    s = torch.cuda.current_stream() if stream is None else stream
    return C.c_void_p(s.cuda_stream) if s.cuda_stream else None


def workspace(device: torch.device, stream: torch.cuda.Stream | None = None) -> torch.Tensor:
    """Zero-initialised verify workspace for (device, stream); kernels leave it zeroed."""
    s = torch.cuda.current_stream(device) if stream is None else stream
    key = (device.index if device.index is not None else torch.cuda.current_device(), s.cuda_stream)
    ws = _workspaces.get(key)
    if ws is None:
        n = int(_lib.lib().wc_workspace_bytes())
        ws = torch.empty((n + 255) // 256 * 256, dtype=torch.uint8, device=device)
        _lib.call("wc_workspace_init", ptr(ws), ws.numel(), stream_ptr(s))
        _workspaces[key] = ws
    return ws


def ptr(t: torch.Tensor | None):
    return None if t is None else C.c_void_p(t.data_ptr())


def i32(x, device) -> torch.Tensor:
    return torch.as_tensor(x, dtype=torch.int32).to(device, non_blocking=False)


def new_verdict(device) -> torch.Tensor:
    """Device buffer holding one wc_verdict (int32 view)."""
    return torch.zeros(_lib.VERDICT_INTS, dtype=torch.int32, device=device)


def reset_workspace(ws: torch.Tensor, stream: torch.cuda.Stream | None = None) -> None:
    """Zero-fill a verify workspace again (after a call reported WC_E_HIP: a
    bounded wait of the one-launch stochastic kernel gave up and left the
    workspace flagged; every later call on it fails fast until this runs)."""
    _lib.call("wc_workspace_init", ptr(ws), ws.numel(), stream_ptr(stream))


def reset_workspaces(device: torch.device | None = None) -> None:
    """reset_workspace for every cached (device, stream) workspace of `device` (None = all)."""
    idx = None if device is None else (device.index if device.index is not None else torch.cuda.current_device())
    for (d, s), ws in _workspaces.items():
        if idx is None or d == idx:
            _lib.call("wc_workspace_init", ptr(ws), ws.numel(), C.c_void_p(s) if s else None)


def check_verdict(out: _lib.Verdict, ws: torch.Tensor | None = None) -> _lib.Verdict:
    """Status of a verdict read back to the host: WC_E_INVALID -> ValueError (the
    device saw an invalid input); WC_E_HIP -> the workspace (`ws`, else every
    cached one) is zero-filled again and RuntimeError is raised."""
    if out.status == _lib.WC_E_HIP:
        if ws is None:
            reset_workspaces()
        else:
            reset_workspace(ws)
        raise _lib.WoodcockHipError("a bounded device-side wait gave up (WC_E_HIP); the verify workspace was "
                                    "re-initialised and this verification has no result")
    if out.status != 0:
        raise ValueError(f"device-side verification rejected its inputs (status {out.status})")
    return out


def read_verdict(v: torch.Tensor, ws: torch.Tensor | None = None) -> _lib.Verdict:
    """The round's host synchronisation: one D2H copy of the verdict."""
    host = v.to("cpu")
    out = _lib.Verdict()
    C.memmove(C.addressof(out), host.numpy().ctypes.data, _lib.VERDICT_BYTES)
    return check_verdict(out, ws)
