"""Type stubs of the neighbour masks: signatures as the registered torch.ops.torchpairwise schemas give them."""
from typing import Optional

from torch import Generator, Tensor

def k_neighbors_mask(x1: Tensor,
                     x2: Optional[Tensor] = None,
                     k: int = 1,
                     metric: str = 'euclidean',
                     *,
                     w: Optional[Tensor] = None,
                     V: Optional[Tensor] = None,
                     VI: Optional[Tensor] = None,
                     p: Optional[float] = None,
                     base: Optional[float] = None,
                     shuffle: Optional[bool] = None,
                     generator: Optional[Generator] = None) -> Tensor: ...


def radius_neighbors_mask(x1: Tensor,
                          x2: Optional[Tensor] = None,
                          epsilon: float = 0.0,
                          metric: str = 'euclidean',
                          *,
                          w: Optional[Tensor] = None,
                          V: Optional[Tensor] = None,
                          VI: Optional[Tensor] = None,
                          p: Optional[float] = None,
                          base: Optional[float] = None,
                          shuffle: Optional[bool] = None,
                          generator: Optional[Generator] = None) -> Tensor: ...
