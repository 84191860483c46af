"""FastGS rasterizer API on PyTorch-ROCm tensors (drop-in for fastgs_core).

Function names, positional order, keyword defaults, dict keys and error
classes follow the reference nanobind module ``_fastgs_core``
(fastgs_core/binding/binding.cpp:512-610).  Arithmetic runs in the HIP
kernels of libfastgs_hip.so; this module validates, allocates outputs with
the torch caching allocator, and wires autograd:

* ``_Preprocess`` mirrors the FastGSPreprocess primitive and its vjp
  (fastgs_preprocess.cpp:41-78, 191-206);
* ``_Rasterize`` mirrors FastGSRasterize and its vjp
  (fastgs_rasterize.cpp:32-88, 191-206).

The ``viewspace_points`` input of ``rasterize_gaussians`` flows into
``_Preprocess`` and its pass-through output into ``_Rasterize``, so the
screen-space gradients (x, y, |x|, |y|) reach the caller's tensor exactly as
on the reference route.

dtype map (reference -> here): uint32 -> torch.int32 (same bits), uint64 ->
torch.int64 (keys < 2^63), bool -> torch.bool, int32/float32 unchanged.
There is no CPU fallback: without a ROCm GPU every entry point raises.
"""
from __future__ import annotations

import ctypes
import threading
import time
from typing import Any, Dict, Optional

import numpy as np
import torch

from . import _lib

TILE = 16

# Whether rasterize_gaussians / rasterize_forward also produce the per-bucket
# sampled state (sample_t / sample_ar).  The backward here does not need it;
# at 1M Gaussians and 1080p it is ~1 GB of writes per forward, so it is off
# unless requested (zero-size tensors are returned otherwise).
WRITE_SAMPLED_STATE = False

# The rasterize backward returns dL/dmeans2d as a view of dL/dviewspace (its
# first two components) instead of a copy; False restores the copy.
MEANS2D_GRAD_VIEW = True

# Optional stage timer (used by bench.py): an object with begin(name) and
# end(name) methods, called around every C-ABI stage on the launch stream.
_STAGE_TIMER = None


def set_stage_timer(timer) -> None:
    """Install (or clear, with None) a timer called around each hot-path stage."""
    global _STAGE_TIMER
    _STAGE_TIMER = timer


class _stage:
    __slots__ = ("name",)

    def __init__(self, name: str):
        self.name = name

    def __enter__(self):
        if _STAGE_TIMER is not None:
            _STAGE_TIMER.begin(self.name)

    def __exit__(self, *exc):
        if _STAGE_TIMER is not None:
            _STAGE_TIMER.end(self.name)
        return False


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------
def _device(t) -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("fastgs_core_amd requires a ROCm GPU (torch.cuda is unavailable); "
                           "there is no CPU fallback")
    if torch.is_tensor(t) and t.is_cuda:
        return t.device
    return torch.device("cuda", torch.cuda.current_device())


def _to(x, dev, dtype) -> Optional[torch.Tensor]:
    if x is None:
        return None
    if not torch.is_tensor(x):
        arr = np.asarray(x)
        if arr.dtype == np.uint64:
            arr = arr.view(np.int64)
        elif arr.dtype == np.uint32:
            arr = arr.view(np.int32)
        x = torch.from_numpy(np.ascontiguousarray(arr))
    if x.dtype in (torch.uint32,):
        x = x.view(torch.int32)
    elif x.dtype in (torch.uint64,):
        x = x.view(torch.int64)
    x = x.to(device=dev, dtype=dtype).contiguous()
    if x.numel() and x.data_ptr() % 16:
        x = x.clone()  # kernels use 8/16-byte vector loads
    return x


def _p(t: Optional[torch.Tensor]):
    """Device pointer of a tensor (None for absent or empty tensors)."""
    if t is None or t.numel() == 0:
        return None
    return t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(dev: torch.device):
    """The current stream of ``dev`` as the C ABI's void* (the raw handle
    lookup skips building a torch Stream object on every call)."""
    if _raw_stream is not None:
        idx = dev.index if dev.index is not None else torch.cuda.current_device()
        return ctypes.c_void_p(_raw_stream(idx))
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


class _SideStreams(threading.local):
    """Per thread and device: the side stream of the colour half of the
    preprocess and its two events (reused from call to call: every call joins
    its colour half before the next one is queued)."""

    def __init__(self):
        self.by_device = {}


_SIDE = _SideStreams()


def _side_stream(dev: torch.device):
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    entry = _SIDE.by_device.get(key)
    if entry is None:
        entry = (torch.cuda.Stream(device=dev), torch.cuda.Event(), torch.cuda.Event())
        _SIDE.by_device[key] = entry
    return entry


def _start_colour(cfg) -> None:
    """Queues the colour half of the preprocess on the side stream, after
    the work queued so far on the current stream."""
    fn = cfg.pop("colour_launch", None)
    if fn is not None:
        fn()


def _join_colour(cfg, dev) -> None:
    """Orders the current stream after the colour half of the preprocess."""
    _start_colour(cfg)
    ev = cfg.get("colour_done")
    if ev is not None:
        torch.cuda.current_stream(dev).wait_event(ev)
        cfg["colour_done"] = None


def _size(x) -> int:
    if x is None:
        return 0
    if torch.is_tensor(x):
        return x.numel()
    return int(np.asarray(x).size)


def _ndim_shape(x):
    if x is None:
        return 0, ()
    if torch.is_tensor(x):
        return x.dim(), tuple(x.shape)
    a = np.asarray(x)
    return a.ndim, a.shape


def _empty_like_path(dev, *shape, dtype=torch.float32):
    return torch.zeros(shape, dtype=dtype, device=dev)


def _tile_bounds(W, H, bx, by):
    return (W + bx - 1) // bx, (H + by - 1) // by, 1


def _check_blocks(bx, by):
    if bx != TILE or by != TILE:
        raise ValueError(f"fastgs_core_amd supports 16x16 tiles only (got {bx}x{by}); the "
                         "reference kernels hard-code BLOCK_X = BLOCK_Y = 16")


def _check_sh(degree: int, max_sh: int, sh_path: bool):
    if sh_path and degree > 0:
        d = min(degree, 3)
        need = (d + 1) ** 2 - 1
        if max_sh < need:
            raise ValueError(f"sh has {max_sh} rest coefficients per Gaussian; degree {degree} "
                             f"needs {need}")


# ---------------------------------------------------------------------------
# autograd Functions
# ---------------------------------------------------------------------------
class _Preprocess(torch.autograd.Function):
    """Preprocess forward + vjp (fastgs_preprocess.cpp:41-78, 191-206)."""

    @staticmethod
    def forward(ctx, cfg, means3d, dc, sh, colors_precomp, opacities, scales, rotations,
                cov3d_precomp, viewmatrix, projmatrix, campos, viewspace_in, log_scales=None,
                raw_rotations=None, opacity_logits=None):
        lib = _lib.load()
        dev = means3d.device
        P = means3d.shape[0]
        f32 = dict(dtype=torch.float32, device=dev)
        # raw: the training scripts' activations are applied inside the
        # preprocess kernels (forward and backward), from the raw parameters
        radii = torch.empty(P, dtype=torch.int32, device=dev)
        xys = torch.empty((P, 2), **f32)
        depths = torch.empty(P, **f32)
        cov3d = torch.empty((P, 6), **f32)
        rgb = torch.empty((P, 3), **f32)
        conic = torch.empty((P, 4), **f32)
        tiles = torch.empty(P, dtype=torch.int32, device=dev)
        clamped = torch.empty((P, 3), dtype=torch.bool, device=dev)
        vsp_out = torch.empty((P, 4), **f32)
        prm = _lib.PreprocessParams(P, cfg["degree"], cfg["max_sh"], cfg["W"], cfg["H"], cfg["gx"],
                                    cfg["gy"], int(cfg["use_cov"]), int(cfg["use_col"]),
                                    cfg["scale_modifier"], cfg["mult"], cfg["tan_fovx"],
                                    cfg["tan_fovy"])
        io = _lib.PreprocessFwdIO(
            _p(means3d), _p(dc), _p(sh), _p(colors_precomp), _p(opacities), _p(scales),
            _p(rotations), _p(cov3d_precomp), _p(viewmatrix), _p(projmatrix), _p(campos),
            _p(viewspace_in), _p(radii), _p(xys), _p(depths), _p(cov3d), _p(rgb), _p(conic),
            _p(tiles), _p(clamped), _p(vsp_out), _p(cfg["st_rec"]), _p(cfg["st_masks"]),
            _p(log_scales), _p(raw_rotations), _p(opacity_logits))
        if P > 0 and cfg.get("split_colour"):
            # geometry on this stream; the colour half on the side stream after
            # it, overlapping the binning (joined before the rasterize)
            with _stage("preprocess_fwd"):
                _lib.check(lib.fgs_preprocess_geometry_fwd(ctypes.byref(prm), ctypes.byref(io),
                                                           _stream(dev)))
            def launch_colour(prm=prm, io=io, keep=(means3d, campos, dc, sh, colors_precomp,
                                                    radii, rgb, clamped)):
                side, start, colour_done = _side_stream(dev)
                start.record(torch.cuda.current_stream(dev))
                side.wait_event(start)
                _lib.check(lib.fgs_preprocess_colour_fwd(ctypes.byref(prm), ctypes.byref(io),
                                                         ctypes.c_void_p(side.cuda_stream)))
                colour_done.record(side)
                for t in keep:
                    if t is not None:
                        t.record_stream(side)
                cfg["colour_done"] = colour_done

            cfg["colour_launch"] = launch_colour
            if COLOUR_START == "geometry":
                _start_colour(cfg)
        elif P > 0:
            with _stage("preprocess_fwd"):
                _lib.check(lib.fgs_preprocess_fwd(ctypes.byref(prm), ctypes.byref(io),
                                                  _stream(dev)))
        ctx.cfg = dict(cfg, st_rec=None, st_masks=None, colour_done=None,
                       colour_launch=None)  # forward-only
        ctx.opacity_shape = (opacity_logits if cfg.get("raw") else opacities).shape
        ctx.sh_shape = None if sh is None else sh.shape
        ctx.save_for_backward(means3d, sh, scales, rotations, cov3d_precomp, viewmatrix,
                              projmatrix, campos, cov3d, radii, clamped, log_scales,
                              raw_rotations, opacity_logits)
        ctx.mark_non_differentiable(radii, tiles, clamped)
        # outputs the loss does not reach arrive as None (no zero tensors)
        ctx.set_materialize_grads(False)
        return radii, xys, depths, cov3d, rgb, conic, tiles, clamped, vsp_out

    @staticmethod
    def backward(ctx, g_radii, g_xys, g_depths, g_cov3d, g_rgb, g_conic, g_tiles, g_clamped,
                 g_vsp):
        lib = _lib.load()
        (means3d, sh, scales, rotations, cov3d_precomp, viewmatrix, projmatrix, campos, cov3d,
         radii, clamped, log_scales, raw_rotations, opacity_logits) = ctx.saved_tensors
        cfg = ctx.cfg
        raw = bool(cfg.get("raw"))
        dev = means3d.device
        P = means3d.shape[0]
        f32 = dict(dtype=torch.float32, device=dev)
        c = lambda g: None if g is None else g.to(torch.float32).contiguous()  # noqa: E731
        # the xy cotangent is read with its row stride when its rows are
        # float pairs (the rasterize backward's view of dL/dviewspace)
        xys_stride = 0
        if (g_xys is not None and g_xys.dtype == torch.float32 and g_xys.dim() == 2
                and g_xys.shape[1] == 2 and g_xys.stride(1) == 1 and g_xys.stride(0) >= 2):
            xys_stride = int(g_xys.stride(0))
        else:
            g_xys = c(g_xys)
        g_rgb, g_conic, g_cov3d, g_vsp = c(g_rgb), c(g_conic), c(g_cov3d), c(g_vsp)
        d_means3d = torch.empty((P, 3), **f32)
        sh_path = not cfg["use_col"]
        d_dc = torch.empty((P, 3), **f32) if sh_path else None
        d_sh = torch.empty(ctx.sh_shape, **f32) if (sh_path and sh is not None) else None
        d_col = torch.empty((P, 3), **f32) if not sh_path else None
        # raw: the gradients of log-scales, raw rotations and opacity logits
        # instead of those of the activated parameters
        d_opac = torch.empty(P, **f32)
        d_scales = torch.empty((P, 3), **f32) if not cfg["use_cov"] else None
        d_rot = torch.empty((P, 4), **f32) if not cfg["use_cov"] else None
        d_vsp = torch.empty((P, 4), **f32)
        prm = _lib.PreprocessParams(P, cfg["degree"], cfg["max_sh"], cfg["W"], cfg["H"], cfg["gx"],
                                    cfg["gy"], int(cfg["use_cov"]), int(cfg["use_col"]),
                                    cfg["scale_modifier"], cfg["mult"], cfg["tan_fovx"],
                                    cfg["tan_fovy"])
        io = _lib.PreprocessBwdIO(
            _p(means3d), _p(scales), _p(rotations), _p(viewmatrix), _p(projmatrix), _p(campos),
            _p(sh), _p(cov3d_precomp), _p(cov3d), _p(radii), _p(clamped), _p(g_xys), _p(g_rgb),
            _p(g_conic), _p(g_cov3d), _p(g_vsp), _p(d_means3d), _p(d_dc), _p(d_sh), _p(d_col),
            None if raw else _p(d_opac), None if raw else _p(d_scales),
            None if raw else _p(d_rot), _p(d_vsp), _p(raw_rotations), None,
            _p(d_scales) if raw else None, _p(d_rot) if raw else None,
            _p(d_opac) if raw else None, _p(log_scales), _p(opacity_logits), xys_stride)
        if P > 0:
            with _stage("preprocess_bwd"):
                _lib.check(lib.fgs_preprocess_bwd(ctypes.byref(prm), ctypes.byref(io),
                                                  _stream(dev)))
        need = ctx.needs_input_grad
        d_cov_pre = torch.zeros_like(cov3d_precomp) if (cov3d_precomp is not None and need[8]) \
            else None
        d_opac = d_opac.view(ctx.opacity_shape)
        act = (None, None, None) if raw else (d_opac, d_scales, d_rot)
        rawg = (d_scales, d_rot, d_opac) if raw else (None, None, None)
        return (None, d_means3d, d_dc, d_sh, d_col, act[0], act[1], act[2], d_cov_pre,
                torch.zeros_like(viewmatrix) if need[9] else None,
                torch.zeros_like(projmatrix) if need[10] else None,
                torch.zeros_like(campos) if need[11] else None, d_vsp) + rawg


class _Rasterize(torch.autograd.Function):
    """Rasterize forward + vjp (fastgs_rasterize.cpp:32-88, 191-206)."""

    @staticmethod
    def forward(ctx, cfg, ranges, point_list, bucket_offsets, means2d, colors, conic_opacity,
                background, radii, metric_map, metric_count, viewspace_points):
        lib = _lib.load()
        dev = means2d.device
        W, H, C, T, B = cfg["W"], cfg["H"], cfg["C"], cfg["T"], cfg["B"]
        P = means2d.shape[0]
        HW = W * H
        f32 = dict(dtype=torch.float32, device=dev)
        ws = bool(cfg["write_sampled"])
        ss = B * 256 if ws else 0
        bucket_to_tile = torch.empty(B, dtype=torch.int32, device=dev)
        sampled_t = torch.empty(ss, **f32)
        sampled_ar = torch.empty((C, ss), **f32)
        final_t = torch.empty(HW, **f32)
        n_contrib = torch.empty(HW, dtype=torch.int32, device=dev)
        max_contrib = torch.empty(T, dtype=torch.int32, device=dev)
        pixel_colors = torch.empty((C, HW), **f32)
        out_color = torch.empty((C, HW), **f32)
        get_flag = bool(cfg["get_flag"])
        mc = torch.zeros(metric_count.shape, dtype=torch.int32, device=dev)
        if get_flag and mc.numel() < P:
            raise ValueError(f"metric_count has {mc.numel()} entries, get_flag needs one per "
                             f"Gaussian ({P})")
        prm = _lib.RasterParams(W, H, C, T, B, int(get_flag), int(ws), P, point_list.numel())
        # optional measurement output (count_iterations): handed back through cfg
        n_iter = torch.empty(HW, dtype=torch.int32, device=dev) if cfg.get("count_iter") else None
        cfg["n_iter"] = n_iter
        io = _lib.RasterFwdIO(
            _p(ranges), _p(point_list), _p(bucket_offsets), _p(means2d), _p(colors),
            _p(conic_opacity), _p(background), _p(metric_map), _p(bucket_to_tile),
            _p(sampled_t), _p(sampled_ar), _p(final_t), _p(n_contrib), _p(max_contrib),
            _p(pixel_colors), _p(out_color), _p(mc), _p(n_iter))
        with _stage("rasterize_fwd"):
            _lib.check(lib.fgs_rasterize_fwd(ctypes.byref(prm), ctypes.byref(io), _stream(dev)))
        ctx.cfg = cfg
        ctx.save_for_backward(ranges, point_list, means2d, colors, conic_opacity, background,
                              final_t, n_contrib, max_contrib)
        ctx.mark_non_differentiable(bucket_to_tile, sampled_t, sampled_ar, final_t, n_contrib,
                                    max_contrib, mc)
        ctx.set_materialize_grads(False)
        return (bucket_to_tile, sampled_t, sampled_ar, final_t, n_contrib, max_contrib,
                pixel_colors, out_color, mc)

    @staticmethod
    def backward(ctx, g_b2t, g_st, g_sar, g_ft, g_nc, g_mc, g_pc, g_out, g_metric):
        lib = _lib.load()
        (ranges, point_list, means2d, colors, conic_opacity, background, final_t, n_contrib,
         max_contrib) = ctx.saved_tensors
        cfg = ctx.cfg
        dev = means2d.device
        W, H, C, T, B = cfg["W"], cfg["H"], cfg["C"], cfg["T"], cfg["B"]
        P = means2d.shape[0]
        f32 = dict(dtype=torch.float32, device=dev)
        if g_out is None:
            g_out = torch.zeros((C, W * H), **f32)
        g_out = g_out.to(torch.float32).contiguous()
        d_colors = torch.empty((P, colors.shape[1] if colors.dim() == 2 else C), **f32)
        d_conic = torch.empty((P, 4), **f32)
        d_vsp = torch.empty((P, 4), **f32)
        # dL/dmeans2d is the first two components of dL/dviewspace: returned
        # as that view (no copy); the preprocess backward reads it in place
        d_means2d = d_vsp[:, :2] if MEANS2D_GRAD_VIEW else torch.empty((P, 2), **f32)
        tile_order = torch.empty(max(T, 1), dtype=torch.int32, device=dev)
        prm = _lib.RasterParams(W, H, C, T, B, 0, 0, P, point_list.numel())
        io = _lib.RasterBwdIO(
            _p(ranges), _p(point_list), _p(means2d), _p(colors), _p(conic_opacity),
            _p(background), _p(final_t), _p(n_contrib), _p(max_contrib), _p(g_out),
            None if MEANS2D_GRAD_VIEW else _p(d_means2d), _p(d_colors), _p(d_conic), _p(d_vsp),
            _p(tile_order))
        with _stage("rasterize_bwd"):
            _lib.check(lib.fgs_rasterize_bwd(ctypes.byref(prm), ctypes.byref(io), _stream(dev)))
        need = ctx.needs_input_grad
        d_bg = torch.zeros_like(background) if need[7] else None
        return (None, None, None, None, d_means2d, d_colors.view(colors.shape), d_conic, d_bg,
                None, None, None, d_vsp)


# ---------------------------------------------------------------------------
# stage helpers shared by the public functions
# ---------------------------------------------------------------------------
def _inclusive_scan_i32(x: torch.Tensor, side=None) -> torch.Tensor:
    """Inclusive scan of x into the first n words of an (n + 1)-word buffer; the
    last word receives the scan's wait status, so one copy of the final two
    words reads the total and the status together.  side: a stream that has
    waited for x, to run the scan on (the buffers are allocated on the current
    stream and marked as used by side)."""
    lib = _lib.load()
    n = x.numel()
    buf = torch.empty(n + 1, dtype=torch.int32, device=x.device)
    ws = torch.empty(int(lib.fgs_scan_workspace_bytes(max(n, 1))), dtype=torch.uint8,
                     device=x.device)
    if side is not None:
        for t in (x, buf, ws):
            t.record_stream(side)
    stream = ctypes.c_void_p(side.cuda_stream) if side is not None else _stream(x.device)
    # the stage timer records on the stream the scan runs on
    with torch.cuda.stream(side if side is not None else torch.cuda.current_stream(x.device)):
        with _stage("scan"):
            _lib.check(lib.fgs_inclusive_scan_u32(_p(x), _p(buf[:n]) if n else None, n, _p(ws),
                                                  _p(buf[n:]), stream))
    return buf


def _binning_sorted(xys, depths, conic, tiles, K: int, gx: int, gy: int, mult: float,
                    depth_ws: Optional[torch.Tensor] = None,
                    st_rec: Optional[torch.Tensor] = None,
                    st_masks: Optional[torch.Tensor] = None, host_word=None):
    lib = _lib.load()
    dev = xys.device
    P = xys.shape[0]
    T = gx * gy
    keys = torch.empty(K, dtype=torch.int64, device=dev)
    plist = torch.empty(K, dtype=torch.int32, device=dev)
    # ranges, counts, offsets, then the wait status next to the last offset (B)
    tbuf = torch.empty(4 * T + 1, dtype=torch.int32, device=dev)
    ranges = tbuf[: 2 * T].view(T, 2)
    bucket_count = tbuf[2 * T: 3 * T]
    bucket_offsets = tbuf[3 * T: 4 * T]
    ws = torch.empty(int(lib.fgs_binning_workspace_bytes(P, K, T)), dtype=torch.uint8, device=dev)
    io = _lib.BinningIO(P, gx, gy, K, mult, _p(xys), _p(depths), _p(conic), _p(tiles), _p(keys),
                        _p(plist), _p(ranges), _p(bucket_count), _p(bucket_offsets), _p(ws),
                        _p(depth_ws), _p(st_rec), _p(st_masks), _p(tbuf[4 * T:]),
                        _p(host_word[0]) if host_word is not None else None)
    with _stage("binning"):
        _lib.check(lib.fgs_binning_sorted(ctypes.byref(io), _stream(dev)))
    return keys, plist, ranges, bucket_count, bucket_offsets, tbuf


class WaitError(RuntimeError):
    """A bounded wait of a scan or sort gave up (see fgs_set_wait_spin_limit);
    the results of that call are invalid."""


def check_wait(status: int, what: str) -> None:
    if status:
        kinds = [k for b, k in ((1, "scan"), (2, "radix look-back")) if status & b]
        raise WaitError(f"{what}: a bounded wait gave up ({', '.join(kinds) or 'unknown'}, "
                        f"wait status {status:#x}); its outputs are invalid")


def _value_and_status(buf: torch.Tensor, i: int):
    """One blocking read of buf[i] (read_last_u32, binding.cpp:25-31) and of the
    wait status stored at buf[i + 1]."""
    a = buf[i:i + 2].cpu().numpy()
    return int(a[0]) & 0xFFFFFFFF, int(a[1]) & 0xFFFFFFFF


class _ReadSlots(threading.local):
    """Per-thread pinned 8-byte slots and events for the asynchronous reads,
    reused from call to call (two can be in flight: K and B)."""

    def __init__(self):
        self.free = []


_READ_SLOTS = _ReadSlots()


def _read_async(buf: torch.Tensor, i: int):
    """read_last_u32 split in two: the copy of buf[i] and the wait status at
    buf[i + 1] to pinned host memory and an event are queued now, the values
    are read by _wait_read.  Work queued in between runs on the GPU while the
    host waits."""
    if _READ_SLOTS.free:
        host, view, ev = _READ_SLOTS.free.pop()
    else:
        host = torch.empty(2, dtype=torch.int32, pin_memory=True)
        view, ev = host.numpy(), torch.cuda.Event()
    host.copy_(buf[i:i + 2], non_blocking=True)
    ev.record(torch.cuda.current_stream(buf.device))
    return host, view, ev


class _HostWords:
    """Pinned 64-bit words the binning writes (status << 32) | B into."""

    def __init__(self):
        self.free = []


_HOST_WORDS = _HostWords()
_HOST_SENTINEL = -1  # low half 0xFFFFFFFF: not written yet


def _host_word():
    """A pinned word set to the sentinel, for fgs_binning_io.host_result."""
    if _HOST_WORDS.free:
        word = _HOST_WORDS.free.pop()
    else:
        t = torch.empty(1, dtype=torch.int64, pin_memory=True)
        word = (t, t.numpy())
    word[1][0] = _HOST_SENTINEL
    return word


def _poll_host_word(word, dev, timeout_s: float = 5.0):
    """(B, status) once the device has written the word.  The value lands
    before the binning's last kernel runs, so the host rarely spins; a word
    still unwritten after timeout_s is read again after the stream has
    drained, then reported as an error."""
    view = word[1]
    v = int(view[0])
    if (v & 0xFFFFFFFF) == 0xFFFFFFFF:
        t0 = time.perf_counter()
        spins = 0
        while (v & 0xFFFFFFFF) == 0xFFFFFFFF:
            el = time.perf_counter() - t0
            if el > timeout_s:
                torch.cuda.current_stream(dev).synchronize()
                v = int(view[0])
                if (v & 0xFFFFFFFF) == 0xFFFFFFFF:
                    raise RuntimeError("fgs_binning_sorted did not write its host result")
                break
            # a tight spin for the first ~50 us (the usual wait), then yield
            # the GIL and the core to the process's other threads
            spins += 1
            if el > 5e-5:
                time.sleep(0 if el < 1e-3 else 1e-4)
            v = int(view[0])
    _HOST_WORDS.free.append(word)
    return v & 0xFFFFFFFF, (v >> 32) & 0xFFFFFFFF


def _wait_read(pending):
    _, view, ev = pending
    ev.synchronize()
    v, st = int(view[0]) & 0xFFFFFFFF, int(view[1]) & 0xFFFFFFFF
    _READ_SLOTS.free.append(pending)
    return v, st


def _count_and_depth_order(scan_buf, depths, tiles, pending=None):
    """K = point_offsets[P-1] (binding.cpp:153-154), read with the scan's wait
    status, and the depth order of the Gaussians, the first stage of the
    binning.  The depth sort needs only P, so it is queued between the copy of
    K and the wait for it."""
    P = tiles.numel()
    if P == 0:
        return 0, None
    lib = _lib.load()
    dev = tiles.device
    if pending is None:  # else the copy is already queued (on the side stream)
        pending = _read_async(scan_buf, P - 1)
    dws = torch.empty(int(lib.fgs_depth_order_workspace_bytes(P)), dtype=torch.uint8, device=dev)
    with _stage("binning"):
        _lib.check(lib.fgs_depth_order(P, _p(depths), _p(tiles), _p(dws), _stream(dev)))
    K, status = _wait_read(pending)
    check_wait(status, "rasterize_gaussians_forward (scan of tiles_touched)")
    return K, dws


# ---------------------------------------------------------------------------
# public API (binding.cpp:512-610)
# ---------------------------------------------------------------------------
def dummy_add(a, b):
    """binding.cpp:514 (build smoke of the reference)."""
    return a + b


def dummy_array_size(a) -> int:
    """binding.cpp:515-518."""
    return int(a.numel()) if torch.is_tensor(a) else int(np.asarray(a).size)


def _colour_and_geometry(inputs: Dict[str, Any], fn: str, col_keys, rot_key: str):
    col = None
    for k in col_keys:
        if _size(inputs.get(k)) != 0:
            col = inputs[k]
            break
    has_dc, has_sh = "dc" in inputs, "sh" in inputs
    has_col = col is not None
    if has_col == (has_dc and has_sh):
        alt = "colors_precomp (or colors)" if len(col_keys) > 1 else "colors_precomp"
        raise RuntimeError(f"{fn} expects exactly one color path: either {alt} OR dc+sh")
    cov = inputs.get("cov3d_precomp")
    has_cov = _size(cov) != 0
    has_sr = _size(inputs.get("scales")) != 0 and _size(inputs.get(rot_key)) != 0
    if has_cov == has_sr:
        raise RuntimeError(f"{fn} expects exactly one geometry path: either cov3d_precomp OR "
                           f"scales+{rot_key}")
    return col, has_col, has_cov


def _run_preprocess(inputs, fn, names, image_width, image_height, block_x, block_y, tan_fovx,
                    tan_fovy, degree, scale_modifier, mult, default_vsp: bool,
                    st_records: bool = False):
    """Shared body of preprocess_forward / rasterize_gaussians (binding.cpp:61-153, 424-492).
    st_records: also write the super-tile records the fused binning reads
    (grids of at most 256 super-tiles of 8x8 tiles)."""
    def req(k):
        if k not in inputs:
            raise RuntimeError(f"{fn} missing required input tensor: {k}")
        return inputs[k]

    # rasterize_gaussians also takes the raw parameters of a training step in
    # place of the activated ones (no reference counterpart): the activations
    # run inside and their backward is fused into the preprocess backward
    raw = names is _RG_NAMES and all(_size(inputs.get(k)) != 0 for k in _RAW_KEYS)
    if raw and any(_size(inputs.get(k)) != 0
                   for k in ("opacities", "scales", "rotations", "cov3d_precomp")):
        raise RuntimeError(f"{fn} takes either opacities/scales/rotations or the raw "
                           f"{'/'.join(_RAW_KEYS)}, not both")
    for k in names["required"]:
        if not (raw and k == "opacities"):
            req(k)
    geo = dict(inputs, scales=inputs["log_scales"], rotations=inputs["raw_rotations"]) if raw \
        else inputs
    col, has_col, has_cov = _colour_and_geometry(geo, fn, names["col_keys"], names["rot"])
    _check_blocks(block_x, block_y)
    sh_nd, sh_shape = _ndim_shape(inputs.get("sh"))
    max_sh = int(sh_shape[1]) if sh_nd >= 2 else 0
    sh_path = not has_col
    _check_sh(degree, max_sh, sh_path)
    dev = _device(inputs[names["means3d"]])
    f = lambda x: _to(x, dev, torch.float32)  # noqa: E731
    means3d = f(inputs[names["means3d"]])
    P = means3d.shape[0]
    opac = f(inputs["opacity_logits" if raw else "opacities"])
    if opac.numel() != P:
        raise ValueError(f"opacities has {opac.numel()} entries for {P} Gaussians")
    if raw:
        ls, rq = f(inputs["log_scales"]), f(inputs["raw_rotations"])
        if ls.shape != (P, 3) or rq.shape != (P, 4):
            raise ValueError(f"{fn} expects log_scales [P,3] and raw_rotations [P,4], got "
                             f"{tuple(ls.shape)} and {tuple(rq.shape)}")
    vsp = inputs.get("viewspace_points")
    if vsp is None or _size(vsp) == 0:
        if not default_vsp:
            raise RuntimeError(f"{fn} missing required input tensor: viewspace_points")
        vsp = torch.zeros((P, 4), dtype=torch.float32, device=dev)
    vsp = f(vsp)
    gx, gy, _ = _tile_bounds(image_width, image_height, block_x, block_y)
    cfg = dict(degree=int(degree), max_sh=max_sh, W=int(image_width), H=int(image_height), gx=gx,
               gy=gy, use_cov=has_cov, use_col=has_col, scale_modifier=float(scale_modifier),
               mult=float(mult), tan_fovx=float(tan_fovx), tan_fovy=float(tan_fovy),
               st_rec=None, st_masks=None, raw=raw, split_colour=bool(st_records and SPLIT_COLOUR),
               colour_done=None)
    if st_records and ((gx + 7) // 8) * ((gy + 7) // 8) <= 256:
        cfg["st_rec"] = torch.empty((P, 4), dtype=torch.int32, device=dev)
        cfg["st_masks"] = torch.empty((P, 4), dtype=torch.int64, device=dev)
    dc = f(inputs["dc"]) if sh_path else None
    sh = f(inputs["sh"]) if sh_path else None
    if sh is not None and sh.numel() == 0:
        sh = sh.reshape(P, 0, 3) if sh.dim() < 3 else sh
    if raw:
        outs = _Preprocess.apply(
            cfg, means3d, dc, sh, f(col) if has_col else None, None, None, None, None,
            f(inputs[names["view"]]), f(inputs[names["proj"]]), f(inputs[names["campos"]]), vsp,
            ls, rq, opac)
        return outs, cfg, dev
    outs = _Preprocess.apply(
        cfg, means3d, dc, sh, f(col) if has_col else None, opac,
        None if has_cov else f(inputs["scales"]), None if has_cov else f(inputs[names["rot"]]),
        f(inputs["cov3d_precomp"]) if has_cov else None, f(inputs[names["view"]]),
        f(inputs[names["proj"]]), f(inputs[names["campos"]]), vsp)
    return outs, cfg, dev


_RAW_KEYS = ("log_scales", "raw_rotations", "opacity_logits")

# rasterize_gaussians runs the preprocess's colour half (the SH colours) on a
# side stream, where it overlaps the binning; False runs the fused kernel.
SPLIT_COLOUR = True
# where the colour half starts on the GPU: right after the geometry half
# ("geometry"), after the scan of tiles_touched ("scan"), or after the depth
# sort, once K is known ("depth")
COLOUR_START = "scan"
# with the colour half split off, the scan of tiles_touched and the copy of K
# also run on the side stream, before the colour half
SCAN_ON_SIDE = True
# B read from a pinned word the binning writes (no copy on the launch stream)
HOST_B = True
_RG_NAMES = dict(required=("means3d", "background", "opacities", "metric_map", "viewmatrix",
                           "projmatrix", "campos"),
                 col_keys=("colors_precomp", "colors"), rot="rotations", means3d="means3d",
                 view="viewmatrix", proj="projmatrix", campos="campos")
_PF_NAMES = dict(required=("means3d", "opacities", "viewmat", "projmat", "cam_pos",
                           "viewspace_points"),
                 col_keys=("colors_precomp",), rot="quats", means3d="means3d", view="viewmat",
                 proj="projmat", campos="cam_pos")


def rasterize_gaussians_forward(inputs: Dict[str, Any], image_width: int, image_height: int,
                                block_x: int = 16, block_y: int = 16, tan_fovx: float = 1.0,
                                tan_fovy: float = 1.0, degree: int = 0,
                                scale_modifier: float = 1.0, mult: float = 1.0,
                                prefiltered: bool = False, get_flag: bool = False,
                                *, write_sampled: Optional[bool] = None,
                                count_iterations: bool = False) -> Dict[str, Any]:
    """Full forward (binding.cpp:33-282): preprocess -> scan -> binning/sort ->
    tile ranges -> bucket offsets -> rasterize.  The two 4-byte reads of the
    reference (K and B) are waited for while the GPU has queued work.

    ``inputs`` may carry, in place of ``opacities``, ``scales`` and
    ``rotations``, the raw parameters of a training step (no reference
    counterpart): ``log_scales`` [P,3], ``raw_rotations`` [P,4] and
    ``opacity_logits`` [P].  The training scripts' activations
    (train_scanner_fixed.py:523-536: exp, q/(|q|+1e-8), sigmoid) are then
    applied inside, and the gradients reach the raw tensors directly: the
    activations' backward is fused into the preprocess backward, with results
    bit-identical to ``activate`` followed by the activated call.

    ``count_iterations`` (measurement, no reference counterpart) adds
    ``img_n_iter``: each pixel's iterations of the reference blend loop
    (fastgs_rasterize.metal:100-131, the stop iteration included)."""
    fn = "rasterize_gaussians_forward"
    outs, cfg, dev = _run_preprocess(inputs, fn, _RG_NAMES, image_width, image_height, block_x,
                                     block_y, tan_fovx, tan_fovy, degree, scale_modifier, mult,
                                     default_vsp=True, st_records=True)
    radii, xys, depths, cov3d, rgb, conic, tiles, clamped, vsp_out = outs
    P = xys.shape[0]
    gx, gy = cfg["gx"], cfg["gy"]
    T = gx * gy
    pending_k = None
    if cfg.get("colour_launch") is not None and SCAN_ON_SIDE and P > 0:
        # the scan and the copy of K on the side stream, then the colour half:
        # the launch stream goes straight on to the depth sort, which needs
        # only the geometry
        side, start, _ = _side_stream(dev)
        start.record(torch.cuda.current_stream(dev))
        side.wait_event(start)
        scan_buf = _inclusive_scan_i32(tiles, side)  # point_offsets, then the wait status
        with torch.cuda.stream(side):
            pending_k = _read_async(scan_buf, P - 1)
            if COLOUR_START == "scan":
                _start_colour(cfg)
    else:
        scan_buf = _inclusive_scan_i32(tiles)  # point_offsets, then the scan's wait status
        if COLOUR_START == "scan":
            _start_colour(cfg)
    point_offsets = scan_buf[:P]
    # the zero-count metric array is made before the wait for K: the host work
    # between K's arrival and the binning launch is on the GPU's critical path
    metric_count = torch.zeros(P if get_flag else 0, dtype=torch.int32, device=dev)
    background = _to(inputs["background"], dev, torch.float32)
    metric_map = _to(inputs["metric_map"], dev, torch.int32)
    K, depth_ws = _count_and_depth_order(scan_buf, depths.detach(), tiles, pending_k)
    _start_colour(cfg)
    point_list_keys = point_list = ranges = bucket_count = bucket_offsets = None
    bucket_to_tile = sampled_t = sampled_ar = final_t = n_contrib = max_contrib = None
    pixel_colors = out_color = None
    B = 0
    if K > 0:
        ws = WRITE_SAMPLED_STATE if write_sampled is None else bool(write_sampled)
        # B without a copy: the binning writes it (with its wait status) into
        # a pinned host word, read after the rasterize launch
        host_word = _host_word() if (HOST_B and not ws and T > 0) else None
        with torch.no_grad():
            (point_list_keys, point_list, ranges, bucket_count, bucket_offsets,
             tbuf) = _binning_sorted(xys.detach(), depths.detach(), conic.detach(), tiles, K, gx,
                                     gy, float(mult), depth_ws, cfg["st_rec"], cfg["st_masks"],
                                     host_word)
        if ws:
            # the sampled state is B * 256 entries: B is needed before the launch
            B, status = _value_and_status(tbuf, 4 * T - 1)
            check_wait(status, "rasterize_gaussians_forward (binning)")
            pending_b = None
        else:
            # B = sum over tiles of ceil(n_t / 32) <= (K + 31 T) / 32: bucket_to_tile
            # is sized by that bound and cut to B once the value arrives, which
            # is waited for after the rasterize launch (with the binning's wait
            # status, the word after it)
            pending_b = host_word if host_word is not None else _read_async(tbuf, 4 * T - 1)
            B = (K + 31 * T) // 32
        if B > 0:
            rcfg = dict(W=cfg["W"], H=cfg["H"], C=3, T=T, B=B, get_flag=bool(get_flag),
                        write_sampled=ws, count_iter=bool(count_iterations))
            _join_colour(cfg, dev)  # the rasterize reads rgb
            (bucket_to_tile, sampled_t, sampled_ar, final_t, n_contrib, max_contrib,
             pixel_colors, out_color, metric_count) = _Rasterize.apply(
                rcfg, ranges, point_list, bucket_offsets, xys, rgb, conic, background, radii,
                metric_map, metric_count, vsp_out)
        if pending_b is not None:
            B, status = (_poll_host_word(pending_b, dev) if host_word is not None
                         else _wait_read(pending_b))
            check_wait(status, "rasterize_gaussians_forward (binning)")
            if bucket_to_tile is not None:
                bucket_to_tile = bucket_to_tile[:B]
    if point_list is None or final_t is None:  # nothing rendered: the reference's empty outputs
        i32 = dict(dtype=torch.int32, device=dev)
        f32 = dict(dtype=torch.float32, device=dev)
        if point_list is None:
            point_list_keys = torch.zeros(0, dtype=torch.int64, device=dev)
            point_list = torch.zeros(0, **i32)
            ranges = torch.zeros((0, 2), **i32)
            bucket_count = torch.zeros(0, **i32)
            bucket_offsets = torch.zeros(0, **i32)
        bucket_to_tile = torch.zeros(0, **i32)
        sampled_t = torch.zeros(0, **f32)
        sampled_ar = torch.zeros(0, **f32)
        final_t = torch.zeros(0, **f32)
        n_contrib = torch.zeros(0, **i32)
        max_contrib = torch.zeros(0, **i32)
        pixel_colors = torch.zeros(0, **f32)
        out_color = torch.zeros(0, **f32)
    _join_colour(cfg, dev)  # before rgb / clamped reach the caller
    result = {
        "rendered": K, "num_buckets": B, "out_color": out_color, "radii": radii,
        "point_offsets": point_offsets, "ranges": ranges, "bucket_count": bucket_count,
        "bucket_offsets": bucket_offsets, "point_list_keys": point_list_keys,
        "point_list": point_list, "metric_count": metric_count, "viewspace_points": vsp_out,
        "geom_means2d": xys, "geom_depths": depths, "geom_cov3d": cov3d, "geom_rgb": rgb,
        "geom_conic_opacity": conic, "geom_tiles_touched": tiles, "geom_clamped": clamped,
        "sample_bucket_to_tile": bucket_to_tile, "sample_t": sampled_t, "sample_ar": sampled_ar,
        "img_final_t": final_t, "img_n_contrib": n_contrib, "img_max_contrib": max_contrib,
        "img_pixel_colors": pixel_colors,
    }
    if count_iterations:
        result["img_n_iter"] = (rcfg["n_iter"] if K > 0 and B > 0 and final_t.numel()
                                else torch.zeros(0, dtype=torch.int32, device=dev))
    return result


rasterize_gaussians = rasterize_gaussians_forward


def preprocess_forward(inputs: Dict[str, Any], image_width: int, image_height: int,
                       block_x: int = 16, block_y: int = 16, tan_fovx: float = 1.0,
                       tan_fovy: float = 1.0, degree: int = 0, scale_modifier: float = 1.0,
                       mult: float = 1.0, prefiltered: bool = False) -> Dict[str, Any]:
    """Preprocess only (binding.cpp:397-508); differentiable."""
    outs, _, _ = _run_preprocess(inputs, "preprocess_forward", _PF_NAMES, image_width,
                                 image_height, block_x, block_y, tan_fovx, tan_fovy, degree,
                                 scale_modifier, mult, default_vsp=False)
    keys = ("radii", "xys", "depths", "cov3d", "rgb", "conic_opacity", "tiles_touched", "clamped",
            "viewspace_points")
    return dict(zip(keys, outs))


def binning_forward(xys, depths, point_offsets, conic_opacity, tiles_touched, mult: float,
                    tile_bounds_x: int, tile_bounds_y: int, tile_bounds_z: int,
                    num_rendered: int) -> Dict[str, Any]:
    """Gaussian-order duplication with keys (binding.cpp:345-375)."""
    lib = _lib.load()
    dev = _device(xys)
    K = int(num_rendered)
    if K == 0:
        return {"point_list_keys_unsorted": torch.zeros(0, dtype=torch.int64, device=dev),
                "point_list_unsorted": torch.zeros(0, dtype=torch.int32, device=dev)}
    xys = _to(xys, dev, torch.float32).detach()
    P = xys.shape[0]
    depths = _to(depths, dev, torch.float32).detach().reshape(-1)
    offs = _to(point_offsets, dev, torch.int32).reshape(-1)
    conic = _to(conic_opacity, dev, torch.float32).detach()
    tiles = _to(tiles_touched, dev, torch.int32).reshape(-1)
    for name, t, n in (("depths", depths, P), ("point_offsets", offs, P),
                       ("conic_opacity", conic, 4 * P), ("tiles_touched", tiles, P)):
        if t.numel() != n:
            raise ValueError(f"binning_forward: {name} has {t.numel()} elements, expected {n}")
    keys = torch.empty(K, dtype=torch.int64, device=dev)
    vals = torch.empty(K, dtype=torch.int32, device=dev)
    _lib.check(lib.fgs_duplicate_with_keys(P, _p(xys), _p(depths), _p(offs), _p(conic), _p(tiles),
                                           float(mult), int(tile_bounds_x), int(tile_bounds_y), K,
                                           _p(keys), _p(vals), _stream(dev)))
    return {"point_list_keys_unsorted": keys, "point_list_unsorted": vals}


def tile_prep_forward(point_list_keys, num_rendered: int, num_tiles: int) -> Dict[str, Any]:
    """Tile ranges + bucket counts (binding.cpp:377-395)."""
    lib = _lib.load()
    dev = _device(point_list_keys)
    T = int(num_tiles)
    if T == 0:
        return {"ranges": torch.zeros((0, 2), dtype=torch.int32, device=dev),
                "bucket_count": torch.zeros(0, dtype=torch.int32, device=dev)}
    keys = _to(point_list_keys, dev, torch.int64).reshape(-1)
    K = min(int(num_rendered), keys.numel())
    ranges = torch.empty((T, 2), dtype=torch.int32, device=dev)
    bc = torch.empty(T, dtype=torch.int32, device=dev)
    _lib.check(lib.fgs_tile_ranges(_p(keys), K, T, _p(ranges), _p(bc), _stream(dev)))
    return {"ranges": ranges, "bucket_count": bc}


def rasterize_forward(ranges, point_list, per_tile_bucket_offset, means2d, colors, conic_opacity,
                      background, radii, metric_map, metric_count, viewspace_points,
                      image_width: int, image_height: int, block_x: int, block_y: int,
                      num_channels: int, num_tiles: int, bucket_sum: int, get_flag: bool = False,
                      *, write_sampled: Optional[bool] = None) -> Dict[str, Any]:
    """Rasterize only (binding.cpp:286-343); differentiable w.r.t. means2d,
    colors, conic_opacity and viewspace_points."""
    _check_blocks(block_x, block_y)
    nd_m, sh_m = _ndim_shape(means2d)
    nd_v, sh_v = _ndim_shape(viewspace_points)
    if nd_m != 2 or sh_m[1] != 2:
        raise ValueError("FastGSRasterize expects means2d with shape (N, 2).")
    if nd_v != 2 or sh_v[1] != 4:
        raise ValueError("FastGSRasterize expects viewspace_points with shape (N, 4).")
    if sh_m[0] != sh_v[0]:
        raise ValueError("FastGSRasterize expects means2d and viewspace_points to share the same N.")
    dev = _device(means2d)
    f = lambda x: _to(x, dev, torch.float32)  # noqa: E731
    i = lambda x: _to(x, dev, torch.int32)  # noqa: E731
    T = int(num_tiles)
    W, H = int(image_width), int(image_height)
    gx, gy, _ = _tile_bounds(W, H, block_x, block_y)
    ranges_t = i(ranges).reshape(-1, 2) if _size(ranges) else torch.zeros((0, 2), dtype=torch.int32,
                                                                            device=dev)
    if ranges_t.shape[0] < min(T, gx * gy):
        raise ValueError(f"rasterize_forward: ranges has {ranges_t.shape[0]} tiles, "
                         f"num_tiles is {T}")
    mc = i(metric_count) if metric_count is not None else torch.zeros(0, dtype=torch.int32,
                                                                        device=dev)
    ws = WRITE_SAMPLED_STATE if write_sampled is None else bool(write_sampled)
    cfg = dict(W=W, H=H, C=int(num_channels), T=T, B=int(bucket_sum), get_flag=bool(get_flag),
               write_sampled=ws)
    colors_t = f(colors)
    outs = _Rasterize.apply(cfg, ranges_t, i(point_list).reshape(-1),
                            i(per_tile_bucket_offset).reshape(-1), f(means2d), colors_t,
                            f(conic_opacity), f(background).reshape(-1), i(radii).reshape(-1),
                            i(metric_map).reshape(-1) if metric_map is not None else None, mc,
                            f(viewspace_points))
    keys = ("bucket_to_tile", "sampled_t", "sampled_ar", "final_t", "n_contrib", "max_contrib",
            "pixel_colors", "out_color", "metric_count")
    return dict(zip(keys, outs))
