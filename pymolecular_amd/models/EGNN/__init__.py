"""EGNN layer modules on the fused HIP kernels (mirror of the reference's models/EGNN)."""
from .egnn_clean import EGNN, E_GCL, get_edges, get_edges_batch, unsorted_segment_mean, unsorted_segment_sum  # noqa
from .layer import EGNN_HIP_Layer, EGNN_Triton_Layer  # noqa: F401
from .forward_kernel import egnn_forward_kernel_node_parallel  # noqa: F401
from .backward_kernel import egnn_backward_kernel_node_parallel  # noqa: F401
from .pytorch_baseline import pytorch_egnn_baseline, swish_torch  # noqa: F401
from .mpnn import MPNN, MPNN_GCL  # noqa: F401
