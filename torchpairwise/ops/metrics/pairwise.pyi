"""Type stubs of the metric ops: signatures as the registered torch.ops.torchpairwise schemas give them."""
from typing import Optional, Tuple

from torch import Generator, Tensor

def euclidean_distances(x1: Tensor,
                        x2: Optional[Tensor] = None) -> Tensor: ...


def haversine_distances(x1: Tensor,
                        x2: Optional[Tensor] = None) -> Tensor: ...


def manhattan_distances(x1: Tensor,
                        x2: Optional[Tensor] = None) -> Tensor: ...


def cosine_distances(x1: Tensor,
                     x2: Optional[Tensor] = None) -> Tensor: ...


def linear_kernel(x1: Tensor,
                  x2: Optional[Tensor] = None) -> Tensor: ...


def polynomial_kernel(x1: Tensor,
                      x2: Optional[Tensor] = None,
                      degree: int = 3,
                      gamma: Optional[float] = None,
                      coef0: float = 1.0) -> Tensor: ...


def sigmoid_kernel(x1: Tensor,
                   x2: Optional[Tensor] = None,
                   gamma: Optional[float] = None,
                   coef0: float = 1.0) -> Tensor: ...


def rbf_kernel(x1: Tensor,
               x2: Optional[Tensor] = None,
               gamma: Optional[float] = None) -> Tensor: ...


def laplacian_kernel(x1: Tensor,
                     x2: Optional[Tensor] = None,
                     gamma: Optional[float] = None) -> Tensor: ...


def cosine_similarity(x1: Tensor,
                      x2: Optional[Tensor] = None) -> Tensor: ...


def additive_chi2_kernel(x1: Tensor,
                         x2: Optional[Tensor] = None) -> Tensor: ...


def chi2_kernel(x1: Tensor,
                x2: Optional[Tensor] = None,
                gamma: float = 1.0) -> Tensor: ...


def directed_hausdorff_distances(x1: Tensor,
                                 x2: Optional[Tensor] = None,
                                 *,
                                 shuffle: bool = False,
                                 generator: Optional[Generator] = None) -> Tuple[Tensor, Tensor, Tensor]: ...


def minkowski_distances(x1: Tensor,
                        x2: Optional[Tensor] = None,
                        p: float = 2.0) -> Tensor: ...


def wminkowski_distances(x1: Tensor,
                         x2: Optional[Tensor] = None,
                         p: float = 2.0,
                         w: Optional[Tensor] = None) -> Tensor: ...


def sqeuclidean_distances(x1: Tensor,
                          x2: Optional[Tensor] = None) -> Tensor: ...


def correlation_distances(x1: Tensor,
                          x2: Optional[Tensor] = None) -> Tensor: ...


def hamming_distances(x1: Tensor,
                      x2: Optional[Tensor] = None) -> Tensor: ...


def jaccard_distances(x1: Tensor,
                      x2: Optional[Tensor] = None) -> Tensor: ...


def kulsinski_distances(x1: Tensor,
                        x2: Optional[Tensor] = None) -> Tensor: ...


def kulczynski1_distances(x1: Tensor,
                          x2: Optional[Tensor] = None) -> Tensor: ...


def seuclidean_distances(x1: Tensor,
                         x2: Optional[Tensor] = None,
                         V: Optional[Tensor] = None) -> Tensor: ...


def cityblock_distances(x1: Tensor,
                        x2: Optional[Tensor] = None) -> Tensor: ...


def mahalanobis_distances(x1: Tensor,
                          x2: Optional[Tensor] = None,
                          VI: Optional[Tensor] = None) -> Tensor: ...


def chebyshev_distances(x1: Tensor,
                        x2: Optional[Tensor] = None) -> Tensor: ...


def braycurtis_distances(x1: Tensor,
                         x2: Optional[Tensor] = None) -> Tensor: ...


def canberra_distances(x1: Tensor,
                       x2: Optional[Tensor] = None) -> Tensor: ...


def jensenshannon_distances(x1: Tensor,
                            x2: Optional[Tensor] = None,
                            base: Optional[float] = None) -> Tensor: ...


def yule_distances(x1: Tensor,
                   x2: Optional[Tensor] = None) -> Tensor: ...


def dice_distances(x1: Tensor,
                   x2: Optional[Tensor] = None) -> Tensor: ...


def rogerstanimoto_distances(x1: Tensor,
                             x2: Optional[Tensor] = None) -> Tensor: ...


def russellrao_distances(x1: Tensor,
                         x2: Optional[Tensor] = None) -> Tensor: ...


def sokalmichener_distances(x1: Tensor,
                            x2: Optional[Tensor] = None) -> Tensor: ...


def sokalsneath_distances(x1: Tensor,
                          x2: Optional[Tensor] = None) -> Tensor: ...


def snr_distances(x1: Tensor,
                  x2: Optional[Tensor] = None) -> Tensor: ...


def l1_distances(x1: Tensor,
                 x2: Optional[Tensor] = None) -> Tensor: ...


def l2_distances(x1: Tensor,
                 x2: Optional[Tensor] = None) -> Tensor: ...


def lp_distances(x1: Tensor,
                 x2: Optional[Tensor] = None,
                 p: float = 2.0) -> Tensor: ...


def linf_distances(x1: Tensor,
                   x2: Optional[Tensor] = None) -> Tensor: ...
