"""Point-cloud neighbourhood search for PyTorch on AMD Instinct MI355X (ROCm).

Drop-in for the neighbourhood-search API of mps_pointops 1.0.0: farthest point
sampling, exact kNN (coordinates and features), first-K ball query,
three_nn/three_interpolate, Chamfer distance, and the torch_cluster-style flat
API.  Tensors live on ``device='cuda'`` (ROCm); each op runs a hand-written
gfx950 kernel from libpointops_hip.so.
"""

from . import flat
from .chamfer import chamfer_distance
from .ops import ball_query, ball_query_multi, fps_ball_knn, furthest_point_sample, knn
from .pointnet2 import three_interpolate, three_nn

__all__ = [
    "ball_query", "ball_query_multi", "chamfer_distance", "flat", "fps_ball_knn", "furthest_point_sample", "knn",
    "three_interpolate", "three_nn",
]
__version__ = "1.0.0"
