import torch

k_neighbors_mask = torch.ops.torchpairwise.k_neighbors_mask
radius_neighbors_mask = torch.ops.torchpairwise.radius_neighbors_mask
