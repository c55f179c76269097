"""cuBladeW8A16LinearLayer (reference: quantization/linear.py:8-137).

INT8 per-output-channel weights with 16-bit activations. On a HIP device
the forward is ONE kernel (cbq_w8a16_linear): MFMA GEMM with the int8 tiles
dequantized in LDS, the scale multiply, the outlier side-GEMM and the bias
add fused into its epilogue. A CPU input keeps the reference's CPU branch
(linear.py:109-110, 127-128: plain torch matmul), which is the reference's
own behaviour for CPU tensors, not a substitute for the HIP path: a HIP input
never runs it, and raises if the HIP library is unavailable.

Storage (buffer names and dtypes as in the reference, linear.py:25-33):
  int8_weights  int8 [out, in]. With outliers, the outlier columns hold 0
                in memory; state_dict() saves the reference's layout (only
                the normal columns, [out, in - n_out]) and load_state_dict
                expands it again. Codes and scales are identical either way:
                a zero column changes no row maximum. Any in - n_out works
                (the reference needs it 16-byte aligned).
  scales        [out] in the layer dtype (fp32 scale rounded to it, :79-81)
  outlier_weights [out, n_out] in the weight's dtype, normal_cols /
                outlier_cols int64 (None without outliers)
  bias          parameter [out] or None
Buffers live on the device of the weight given to quantize() (the reference
copies them back to CPU, so every forward re-uploaded the weight).
"""
from __future__ import annotations

import torch
import torch.nn as nn

from .outlier_utils import detect_activation_outlier_columns, detect_outlier_columns
from .quantizers import quantize_tensor
from cublade_amd.bindings.hip.w8a16 import w8a16_linear


class cuBladeW8A16LinearLayer(nn.Module):
    def __init__(
        self,
        in_features,
        out_features,
        bias=True,
        dtype=torch.bfloat16,
        handle_outliers=False,
        outlier_threshold=6.0,
        outlier_mode="weight",
    ):
        super().__init__()
        if outlier_mode not in ("weight", "activation"):
            raise ValueError(f"outlier_mode must be 'weight' or 'activation', got {outlier_mode!r}")
        self.in_features = in_features
        self.out_features = out_features
        self.handle_outliers = handle_outliers
        self.outlier_threshold = outlier_threshold
        self.outlier_mode = outlier_mode
        self.register_buffer("int8_weights",
                             torch.empty(out_features, in_features, dtype=torch.int8))
        self.register_buffer("scales", torch.ones(out_features, dtype=dtype))
        self.register_buffer("outlier_weights", None)
        self.register_buffer("normal_cols", None)
        self.register_buffer("outlier_cols", None)
        self.bias = nn.Parameter(torch.zeros(out_features, dtype=dtype)) if bias else None

    @torch.no_grad()
    def quantize(self, weight_fp: torch.Tensor, activations: torch.Tensor | None = None):
        """Quantize a [out, in] weight per output channel (INT8, symmetric).

        With handle_outliers, the outlier columns are kept in the weight's
        dtype for the side-GEMM and zeroed in the INT8 copy (so their scales
        come from the normal columns only, as in linear.py:48-66). Which
        columns: outlier_mode "weight" (the reference's rule, the default):
        any |w| > outlier_threshold in the column; "activation" (opt-in,
        LLM.int8's rule): any |x| > outlier_threshold in that input feature
        of `activations`, a calibration batch [..., in_features] that this
        mode requires. The quantization itself runs on the GPU.
        """
        if self.handle_outliers and self.outlier_mode == "activation" and (
                activations is None or activations.shape[-1] != self.in_features):
            raise ValueError("outlier_mode='activation' needs a calibration batch "
                             f"[..., {self.in_features}] passed as activations=")
        home = weight_fp.device
        w = weight_fp.detach()
        w = (w if w.is_cuda else w.cuda()).contiguous()
        if tuple(w.shape) != (self.out_features, self.in_features):
            raise ValueError(f"weight must be [{self.out_features}, {self.in_features}], "
                             f"got {tuple(w.shape)}")
        if self.handle_outliers:
            if self.outlier_mode == "activation":
                outlier_cols = detect_activation_outlier_columns(activations,
                                                                 self.outlier_threshold)
            else:
                outlier_cols = detect_outlier_columns(w, threshold=self.outlier_threshold)
            outlier_set = set(outlier_cols)
            normal_cols = [c for c in range(self.in_features) if c not in outlier_set]
            self.outlier_weights = w[:, outlier_cols].to(home)
            self.normal_cols = torch.tensor(normal_cols, dtype=torch.long, device=home)
            self.outlier_cols = torch.tensor(outlier_cols, dtype=torch.long, device=home)
            if outlier_cols:
                w = w.clone()
                w[:, outlier_cols] = 0
        qt = quantize_tensor(w, scheme="symmetric", dtype=torch.int8, mode="channel", ch_axis=0)
        assert torch.count_nonzero(qt.zero_point).item() == 0, "Expect symmetric zp=0"
        scale_1d = qt.scale.squeeze()
        assert scale_1d.ndim == 1 and scale_1d.numel() == self.out_features
        self.int8_weights = qt.data.to(home)
        self.scales = scale_1d.to(device=home, dtype=self.scales.dtype)

    def _outliers_active(self) -> bool:
        return (self.handle_outliers and self.outlier_cols is not None
                and self.outlier_cols.numel() > 0)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        orig_shape = x.shape
        x2d = x.reshape(-1, self.in_features)
        outliers = self._outliers_active()
        if x2d.is_cuda:
            y2d = w8a16_linear(
                x2d, self.int8_weights, self.scales, self.bias,
                self.outlier_cols if outliers else None,
                self.outlier_weights if outliers else None,
            )
        else:
            y2d = self._forward_cpu(x2d, outliers)
        return y2d.view(*orig_shape[:-1], self.out_features)

    def _forward_cpu(self, x2d: torch.Tensor, outliers: bool) -> torch.Tensor:
        """The reference's CPU branch (linear.py:97-135) for CPU tensors."""
        w = self.int8_weights.to(dtype=x2d.dtype, device=x2d.device)
        y2d = (x2d @ w.t()) * self.scales.to(dtype=x2d.dtype, device=x2d.device)
        if outliers:
            idx = self.outlier_cols.to(x2d.device)
            w_out = self.outlier_weights.to(dtype=x2d.dtype, device=x2d.device)
            y2d = y2d + x2d[:, idx] @ w_out.t()
        if self.bias is not None:
            y2d = y2d + self.bias.to(y2d.dtype)
        return y2d

    def _save_to_state_dict(self, destination, prefix, keep_vars):
        # Save the reference's layout (linear.py:48-66): with outliers,
        # int8_weights holds only the normal columns, [out, in - n_out].
        super()._save_to_state_dict(destination, prefix, keep_vars)
        key = prefix + "int8_weights"
        if key in destination and self.normal_cols is not None and self.outlier_cols is not None \
                and self.outlier_cols.numel() > 0:
            wq = destination[key]
            destination[key] = wq[:, self.normal_cols.to(wq.device)].contiguous()

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys,
                              unexpected_keys, error_msgs):
        # Outlier buffers are None in a fresh layer: adopt them from the
        # state dict, and expand the reference's compact [out, in - n_out]
        # int8_weights to [out, in] with zero outlier columns.
        for name in ("outlier_weights", "normal_cols", "outlier_cols"):
            key = prefix + name
            if key in state_dict and getattr(self, name) is None:
                setattr(self, name, state_dict[key].clone())
        key = prefix + "int8_weights"
        if key in state_dict and self.normal_cols is not None:
            wq = state_dict[key]
            n_normal = self.normal_cols.numel()
            if wq.dim() == 2 and wq.size(1) == n_normal and n_normal != self.in_features:
                full = torch.zeros(wq.size(0), self.in_features, dtype=wq.dtype, device=wq.device)
                full[:, self.normal_cols.to(wq.device)] = wq
                state_dict[key] = full
        key = prefix + "int8_weights"
        if key in state_dict and tuple(state_dict[key].shape) != tuple(self.int8_weights.shape):
            self.int8_weights = torch.empty_like(state_dict[key])
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys,
                                      unexpected_keys, error_msgs)


# Lower-case alias of the reference class name.
cubladeW8A16LinearLayer = cuBladeW8A16LinearLayer
