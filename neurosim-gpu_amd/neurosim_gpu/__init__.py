"""NeuroSim dendritic tick on AMD Instinct MI355X (gfx950).

The package keeps the public API of NeuroSim-GPU's dendritic mainline
(DendriticDynamics, the matrix and PELS runtimes, their native variants,
SparseTopology / random_topology, precision codecs, checkpoint/resume) and runs
the native tick as hand-written HIP kernels behind the C ABI declared in
include/neurosim_hip.h (library: neurosim_gpu/_lib/libneurosim_hip.so).
"""

from .checkpoint import (capture_runtime, load_runtime_checkpoint, restore_runtime,
                         save_runtime_checkpoint)
from .compartmental import DendriticDynamics, DendriticMatrixRuntime, DendriticPELSRuntime
from .dynamics import Dynamics
from .native import load_native_extension
from .native_compartmental import NativeDendriticMatrixRuntime, NativeDendriticPELSRuntime
from .precision import PRECISIONS, encode_sparse_weights, quantize_dequantize
from .rollout import MatrixRollout
from .runtime import DenseOracle, HybridPELSRuntime, MatrixRuntime, RuntimeStats
from .topology import SparseTopology, random_topology, topology_to
from .topology_io import load_topology, save_topology, topology_from_dict, topology_to_dict

__version__ = "0.1.0"

__all__ = [
    "DendriticDynamics", "DendriticMatrixRuntime", "DendriticPELSRuntime", "DenseOracle",
    "Dynamics", "HybridPELSRuntime", "MatrixRollout", "MatrixRuntime",
    "NativeDendriticMatrixRuntime", "NativeDendriticPELSRuntime", "PRECISIONS", "RuntimeStats",
    "SparseTopology", "capture_runtime", "encode_sparse_weights", "load_native_extension",
    "load_runtime_checkpoint", "load_topology", "quantize_dequantize", "random_topology",
    "restore_runtime", "save_runtime_checkpoint", "save_topology", "topology_from_dict",
    "topology_to", "topology_to_dict",
]
