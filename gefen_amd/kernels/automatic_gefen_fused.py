"""Fused update entry points (reference: kernels/automatic_gefen_fused.py).

Same names, argument order, checks and exception types as the reference
wrappers (automatic_gefen_fused.py:10-489); the work runs in libgefen_hip.so on
torch's current HIP stream.  The arithmetic is the reference's CPU path, so the
indices and magnitudes these write equal the ``fused=False`` optimizer's.
"""

from __future__ import annotations

import torch

from .gefen_hip import check, device_guard, dtype_code, load_extension, stream_of

_STATE_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def _check_devices(tensors) -> None:
    for name, tensor in tensors.items():
        if not isinstance(tensor, torch.Tensor):
            raise TypeError("Expected {} to be a torch.Tensor.".format(name))
        elif tensor.device.type != "cuda":
            raise ValueError("Expected {} to be on CUDA, got device {}.".format(name, tensor.device))


def _require_contiguous(**tensors) -> None:
    for name, t in tensors.items():
        if not t.is_contiguous():
            raise ValueError("Expected {} to be contiguous.".format(name))


def _check_common_blocks(grad_view, p, m_sign, m_magnitude, codebook, packed_indices):
    if grad_view.dim() != 2:
        raise ValueError("Expected grad_view to be 2D, got dim={}".format(grad_view.dim()))
    elif grad_view.dtype != p.dtype:
        raise ValueError("Expected grad_view dtype {} to match p dtype {}.".format(grad_view.dtype, p.dtype))
    elif m_magnitude.dim() != 2 or m_magnitude.shape[1] != 1:
        raise ValueError("Expected m_magnitude to have shape [num_blocks, 1], got {}".format(
            tuple(m_magnitude.shape)))


def _check_tail(grad_view, m_sign, m_magnitude, codebook, packed_indices):
    if m_sign.dtype != torch.uint8:
        raise ValueError("Expected m_sign to be uint8, got {}".format(m_sign.dtype))
    elif m_magnitude.dtype not in _STATE_DTYPES:
        raise ValueError("Expected m_magnitude to be float32, float16, or bfloat16, got {}".format(m_magnitude.dtype))
    elif codebook.dtype != torch.float32:
        raise ValueError("Expected codebook to be float32, got {}".format(codebook.dtype))
    elif codebook.numel() > 256:
        raise ValueError("Expected codebook to have at most 256 entries, got {}".format(codebook.numel()))
    elif packed_indices and m_sign.numel() != (grad_view.numel() + 1) // 2:
        raise ValueError("Expected packed m_sign.numel()={} for grad_view.numel()={}, got {}.".format(
            (grad_view.numel() + 1) // 2, grad_view.numel(), m_sign.numel()))
    elif not packed_indices and m_sign.numel() != grad_view.numel():
        raise ValueError("Expected unpacked m_sign.numel()={} for grad_view.numel()={}, got {}.".format(
            grad_view.numel(), grad_view.numel(), m_sign.numel()))


def automatic_gefen_fused_update_cuda(p, grad_view, m_sign, m_magnitude, stepsize, codebook,
                                      packed_indices: bool, beta1: float, lr: float) -> None:
    """automatic_gefen_fused.py:10-117: update with a given fp32 stepsize per block."""
    _check_devices({"p": p, "grad_view": grad_view, "m_sign": m_sign, "m_magnitude": m_magnitude,
                    "stepsize": stepsize, "codebook": codebook})
    _check_common_blocks(grad_view, p, m_sign, m_magnitude, codebook, packed_indices)
    if stepsize.dim() != 2 or stepsize.shape[1] != 1:
        raise ValueError("Expected stepsize to have shape [num_blocks, 1], got {}".format(tuple(stepsize.shape)))
    elif grad_view.shape[0] != m_magnitude.shape[0]:
        raise ValueError("Expected grad_view and m_magnitude to have the same number of blocks.")
    elif grad_view.shape[0] != stepsize.shape[0]:
        raise ValueError("Expected grad_view and stepsize to have the same number of blocks.")
    elif m_sign.dtype != torch.uint8:
        raise ValueError("Expected m_sign to be uint8, got {}".format(m_sign.dtype))
    elif m_magnitude.dtype not in _STATE_DTYPES:
        raise ValueError("Expected m_magnitude to be float32, float16, or bfloat16, got {}".format(m_magnitude.dtype))
    elif stepsize.dtype != torch.float32:
        raise ValueError("Expected stepsize to be float32, got {}".format(stepsize.dtype))
    _check_tail(grad_view, m_sign, m_magnitude, codebook, packed_indices)
    lib = load_extension()
    g = grad_view.contiguous()
    st = stepsize.contiguous()
    cb = codebook.contiguous()
    _require_contiguous(p=p, m_sign=m_sign, m_magnitude=m_magnitude)
    if p.numel() != g.numel():
        raise ValueError("Expected p.numel() to match grad_view.numel().")
    with device_guard(p):
        rc = lib.gefen_automatic_fused_update(
            p.data_ptr(), g.data_ptr(), dtype_code(p.dtype), m_sign.data_ptr(), m_magnitude.data_ptr(),
            dtype_code(m_magnitude.dtype), st.data_ptr(), cb.data_ptr(), cb.numel(), int(bool(packed_indices)),
            g.shape[0], g.shape[1], float(beta1), float(lr), stream_of(p))
    check(rc, "automatic_gefen_fused_update_cuda")


def automatic_gefen_fused_update_from_vmean_cuda(p, grad_view, m_sign, m_magnitude, vmean, codebook,
                                                 packed_indices: bool, beta1: float, lr: float,
                                                 bias_correction_1: float, bias_correction_2: float,
                                                 eps: float) -> None:
    """automatic_gefen_fused.py:120-249: stepsize from the updated vmean (gefen.py:1326-1327)."""
    _check_devices({"p": p, "grad_view": grad_view, "m_sign": m_sign, "m_magnitude": m_magnitude,
                    "vmean": vmean, "codebook": codebook})
    _check_common_blocks(grad_view, p, m_sign, m_magnitude, codebook, packed_indices)
    if vmean.dim() != 2 or vmean.shape[1] != 1:
        raise ValueError("Expected vmean to have shape [num_blocks, 1], got {}".format(tuple(vmean.shape)))
    elif grad_view.shape[0] != m_magnitude.shape[0]:
        raise ValueError("Expected grad_view and m_magnitude to have the same number of blocks.")
    elif grad_view.shape[0] != vmean.shape[0]:
        raise ValueError("Expected grad_view and vmean to have the same number of blocks.")
    _check_tail(grad_view, m_sign, m_magnitude, codebook, packed_indices)
    if vmean.dtype not in _STATE_DTYPES:
        raise ValueError("Expected vmean to be float32, float16, or bfloat16, got {}".format(vmean.dtype))
    elif bias_correction_1 <= 0.0:
        raise ValueError("Expected bias_correction_1 to be positive, got {}".format(bias_correction_1))
    elif bias_correction_2 <= 0.0:
        raise ValueError("Expected bias_correction_2 to be positive, got {}".format(bias_correction_2))
    elif eps < 0.0:
        raise ValueError("Expected eps to be non-negative, got {}".format(eps))
    lib = load_extension()
    g = grad_view.contiguous()
    v = vmean.contiguous()
    cb = codebook.contiguous()
    _require_contiguous(p=p, m_sign=m_sign, m_magnitude=m_magnitude)
    if p.numel() != g.numel():
        raise ValueError("Expected p.numel() to match grad_view.numel().")
    with device_guard(p):
        rc = lib.gefen_automatic_fused_update_from_vmean(
            p.data_ptr(), g.data_ptr(), dtype_code(p.dtype), m_sign.data_ptr(), m_magnitude.data_ptr(),
            dtype_code(m_magnitude.dtype), v.data_ptr(), dtype_code(v.dtype), cb.data_ptr(), cb.numel(),
            int(bool(packed_indices)), g.shape[0], g.shape[1], float(beta1), float(lr),
            float(bias_correction_1), float(bias_correction_2), float(eps), stream_of(p))
    check(rc, "automatic_gefen_fused_update_from_vmean_cuda")


def automatic_gefen_period1_update_cuda(p, grad_flat, m_sign, m_magnitude, vmean, codebook,
                                        period_one_divisor: int, beta1: float, beta2: float, lr: float,
                                        bias_correction_1: float, bias_correction_2: float, eps: float) -> None:
    """automatic_gefen_fused.py:252-388: period-1 update with per-element vmean."""
    _check_devices({"p": p, "grad_flat": grad_flat, "m_sign": m_sign, "m_magnitude": m_magnitude,
                    "vmean": vmean, "codebook": codebook})
    if grad_flat.dim() != 1:
        raise ValueError("Expected grad_flat to be 1D, got dim={}".format(grad_flat.dim()))
    elif grad_flat.dtype != p.dtype:
        raise ValueError("Expected grad_flat dtype {} to match p dtype {}.".format(grad_flat.dtype, p.dtype))
    elif p.numel() != grad_flat.numel():
        raise ValueError("Expected p.numel() to match grad_flat.numel().")
    elif m_sign.dtype != torch.uint8:
        raise ValueError("Expected m_sign to be uint8, got {}".format(m_sign.dtype))
    elif m_sign.numel() != grad_flat.numel():
        raise ValueError("Expected m_sign.numel() to match grad_flat.numel().")
    elif m_magnitude.dim() != 2 or m_magnitude.shape[1] != 1:
        raise ValueError("Expected m_magnitude to have shape [num_magnitude_blocks, 1], got {}".format(
            tuple(m_magnitude.shape)))
    elif vmean.dim() != 2 or vmean.shape[1] != 1:
        raise ValueError("Expected vmean to have shape [numel, 1], got {}".format(tuple(vmean.shape)))
    elif not isinstance(period_one_divisor, int):
        raise TypeError("Expected period_one_divisor to be an int, got {}".format(type(period_one_divisor).__name__))
    elif period_one_divisor <= 0:
        raise ValueError("Expected period_one_divisor to be positive, got {}".format(period_one_divisor))
    elif grad_flat.numel() % period_one_divisor != 0:
        raise ValueError("Expected period_one_divisor {} to divide grad_flat.numel() {}.".format(
            period_one_divisor, grad_flat.numel()))
    elif m_magnitude.shape[0] != grad_flat.numel() // period_one_divisor:
        raise ValueError("Expected m_magnitude to have one row per period-one magnitude block.")
    elif vmean.shape[0] != grad_flat.numel():
        raise ValueError("Expected vmean to have one row per gradient element.")
    elif m_magnitude.dtype not in _STATE_DTYPES:
        raise ValueError("Expected m_magnitude to be float32, float16, or bfloat16, got {}".format(m_magnitude.dtype))
    elif vmean.dtype not in _STATE_DTYPES:
        raise ValueError("Expected vmean to be float32, float16, or bfloat16, got {}".format(vmean.dtype))
    elif codebook.dtype != torch.float32:
        raise ValueError("Expected codebook to be float32, got {}".format(codebook.dtype))
    elif codebook.numel() > 256:
        raise ValueError("Expected codebook to have at most 256 entries, got {}".format(codebook.numel()))
    elif not 0.0 <= beta2 <= 1.0:
        raise ValueError("Expected beta2 to be in [0, 1], got {}".format(beta2))
    elif bias_correction_1 <= 0.0:
        raise ValueError("Expected bias_correction_1 to be positive, got {}".format(bias_correction_1))
    elif bias_correction_2 <= 0.0:
        raise ValueError("Expected bias_correction_2 to be positive, got {}".format(bias_correction_2))
    elif eps < 0.0:
        raise ValueError("Expected eps to be non-negative, got {}".format(eps))
    lib = load_extension()
    g = grad_flat.contiguous()
    cb = codebook.contiguous()
    _require_contiguous(p=p, m_sign=m_sign, m_magnitude=m_magnitude, vmean=vmean)
    with device_guard(p):
        rc = lib.gefen_automatic_period1_update(
            p.data_ptr(), g.data_ptr(), dtype_code(p.dtype), m_sign.data_ptr(), m_magnitude.data_ptr(),
            dtype_code(m_magnitude.dtype), vmean.data_ptr(), dtype_code(vmean.dtype), cb.data_ptr(), cb.numel(),
            g.numel(), period_one_divisor, float(beta1), float(beta2), float(lr), float(bias_correction_1),
            float(bias_correction_2), float(eps), stream_of(p))
    check(rc, "automatic_gefen_period1_update_cuda")


def automatic_gefen_muon_momentum_cuda(grad_view, m_sign, m_magnitude, codebook, momentum_update,
                                       packed_indices: bool, beta1: float) -> None:
    """automatic_gefen_fused.py:391-489: quantised GefenMuon momentum, dequantised into momentum_update."""
    _check_devices({"grad_view": grad_view, "m_sign": m_sign, "m_magnitude": m_magnitude,
                    "codebook": codebook, "momentum_update": momentum_update})
    if grad_view.dim() != 2:
        raise ValueError("Expected grad_view to be 2D, got dim={}".format(grad_view.dim()))
    elif momentum_update.shape != grad_view.shape:
        raise ValueError("Expected momentum_update shape {} to match grad_view shape {}.".format(
            tuple(momentum_update.shape), tuple(grad_view.shape)))
    elif momentum_update.dtype != grad_view.dtype:
        raise ValueError("Expected momentum_update dtype {} to match grad_view dtype {}.".format(
            momentum_update.dtype, grad_view.dtype))
    elif m_magnitude.dim() != 2 or m_magnitude.shape[1] != 1:
        raise ValueError("Expected m_magnitude to have shape [num_blocks, 1], got {}".format(
            tuple(m_magnitude.shape)))
    elif grad_view.shape[0] != m_magnitude.shape[0]:
        raise ValueError("Expected grad_view and m_magnitude to have the same number of blocks.")
    _check_tail(grad_view, m_sign, m_magnitude, codebook, packed_indices)
    if not 0.0 <= beta1 < 1.0:
        raise ValueError("Expected beta1 to be in [0, 1), got {}".format(beta1))
    lib = load_extension()
    g = grad_view.contiguous()
    cb = codebook.contiguous()
    _require_contiguous(m_sign=m_sign, m_magnitude=m_magnitude, momentum_update=momentum_update)
    with device_guard(g):
        rc = lib.gefen_automatic_muon_momentum(
            g.data_ptr(), dtype_code(g.dtype), m_sign.data_ptr(), m_magnitude.data_ptr(),
            dtype_code(m_magnitude.dtype), cb.data_ptr(), cb.numel(), momentum_update.data_ptr(),
            int(bool(packed_indices)), g.shape[0], g.shape[1], float(beta1), stream_of(g))
    check(rc, "automatic_gefen_muon_momentum_cuda")
