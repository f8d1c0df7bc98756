"""Neurocell v2 VNN propagation step on AMD Instinct MI355X (gfx950).

Public names mirror the reference package's exports (neurocell/__init__.py:14-88) for the
propagation path: topology, parameters and the Codd fusion, the spectral Green's
correlation operators, the fused epilogues, propagation, adaptive bucketing, the model and
the trainer.  Every operator runs on hand-written HIP kernels behind the C ABI in
``include/neurocell_hip.h`` (``libneurocell_hip.so``, loaded on first use).
"""
__version__ = "1.0.0"

from .topology import ChipTopology2D, CoordinatePortSpec, PortSpec
from .params import (STATE_ACTIVE, STATE_ACTIVE_VALUE, STATE_SIGNAL, STATE_SIGNAL_VALUE,
                     SUPPORTED_CODD_MODES, PrecomputedStepParams, VNNParams,
                     compute_codd_state_probs, init_vnn_params, precompute_step_params)
from .ops import (conv2d_batched_nchw, conv2d_grouped_filter_grad, conv2d_hybrid_nopad_roi_step,
                  conv2d_hybrid_roi_step, conv2d_pruned_rfft_roi_step, conv2d_roi_rfft_step,
                  conv2d_small_kernel_roi_step, conv2d_valid_rfft_precomputed,
                  fused_output_port_epilogue, fused_roi_epilogue, fused_roi_step_epilogue,
                  hoist_filter_rfft2, hoist_filter_rfft2_nopad, hoist_filter_rfft2_zero_fwd,
                  hoist_filter_rfft2_zero_nopad, irfft2_pruned, is_supported_pallas_activation,
                  pallas_fused_output_port_epilogue, pallas_fused_roi_step_epilogue,
                  pallas_standardize_output_port, precompute_filter_rfft2,
                  rfft2_filter_grad_to_oihw, rfft2_pruned, rfft2_unshifted_filter_grad_to_oihw,
                  standardize_spatial_nchw)
from .propagator import (SUPPORTED_BACKENDS, inject_inputs_2d, inject_inputs_roi_2d,
                         propagate_vnn_2d, select_optimal_backend)
from .adaptive_mask import (AdaptiveMaskSpec, compute_adaptive_spatial_mask,
                            estimate_effective_filter_radii)
from .model import VonNeumannNetwork
from .datasets import (ALUDeviceDataset, alu_truth_table, generate_arithmetic,
                       generate_arithmetic_logic, prepare_alu_device_dataset)
from .trainer import (AdamW, AdamWState, VNNTrainer, adamw, compute_annealed_temperature,
                      constant_schedule, cosine_decay_schedule, default_exact_match_metric,
                      default_mse_loss, linear_schedule, packbits_u8_on_device,
                      warmup_cosine_decay_schedule)
from ._lib import NeurocellError

__all__ = [
    "PortSpec", "CoordinatePortSpec", "ChipTopology2D",
    "STATE_ACTIVE", "STATE_SIGNAL", "STATE_ACTIVE_VALUE", "STATE_SIGNAL_VALUE",
    "SUPPORTED_CODD_MODES", "VNNParams", "PrecomputedStepParams", "compute_codd_state_probs",
    "init_vnn_params", "precompute_step_params",
    "rfft2_pruned", "irfft2_pruned", "conv2d_grouped_filter_grad", "conv2d_batched_nchw",
    "precompute_filter_rfft2", "rfft2_filter_grad_to_oihw", "hoist_filter_rfft2",
    "conv2d_roi_rfft_step", "conv2d_valid_rfft_precomputed", "hoist_filter_rfft2_zero_fwd",
    "conv2d_hybrid_roi_step", "rfft2_unshifted_filter_grad_to_oihw",
    "is_supported_pallas_activation", "pallas_fused_roi_step_epilogue",
    "pallas_standardize_output_port", "pallas_fused_output_port_epilogue",
    "hoist_filter_rfft2_nopad", "hoist_filter_rfft2_zero_nopad", "conv2d_hybrid_nopad_roi_step",
    "conv2d_small_kernel_roi_step", "conv2d_pruned_rfft_roi_step",
    "standardize_spatial_nchw", "fused_roi_step_epilogue", "fused_roi_epilogue",
    "fused_output_port_epilogue",
    "SUPPORTED_BACKENDS", "select_optimal_backend", "inject_inputs_2d", "inject_inputs_roi_2d",
    "propagate_vnn_2d",
    "AdaptiveMaskSpec", "estimate_effective_filter_radii", "compute_adaptive_spatial_mask",
    "VonNeumannNetwork",
    "ALUDeviceDataset", "generate_arithmetic", "generate_arithmetic_logic",
    "prepare_alu_device_dataset", "alu_truth_table",
    "VNNTrainer", "AdamW", "AdamWState", "adamw", "constant_schedule", "linear_schedule",
    "cosine_decay_schedule", "warmup_cosine_decay_schedule", "compute_annealed_temperature",
    "packbits_u8_on_device", "default_mse_loss", "default_exact_match_metric",
    "NeurocellError",
]
