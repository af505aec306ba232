import torch

cdist = torch.ops.torchpairwise.cdist
pdist = torch.ops.torchpairwise.pdist
