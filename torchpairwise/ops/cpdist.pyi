"""Type stubs of cdist / pdist: signatures as the registered torch.ops.torchpairwise schemas give them."""
from typing import Optional

from torch import Generator, Tensor

def cdist(x1: Tensor,
          x2: Tensor,
          metric: str = 'minkowski',
          *,
          w: Optional[Tensor] = None,
          V: Optional[Tensor] = None,
          VI: Optional[Tensor] = None,
          p: Optional[float] = None,
          base: Optional[float] = None,
          shuffle: Optional[bool] = None,
          generator: Optional[Generator] = None) -> Tensor: ...


def pdist(input: Tensor,
          metric: str = 'minkowski',
          *,
          w: Optional[Tensor] = None,
          V: Optional[Tensor] = None,
          VI: Optional[Tensor] = None,
          p: Optional[float] = None,
          base: Optional[float] = None,
          shuffle: Optional[bool] = None,
          generator: Optional[Generator] = None) -> Tensor: ...
