"""Module-level bindings of the ops (reference: torchpairwise/ops/metrics/pairwise.py:4-47,
ops/cpdist.py:3-4, ops/metrics/neighbors.py:3-4)."""
import torch

_METRICS = [
    # sklearn
    "euclidean_distances", "haversine_distances", "manhattan_distances", "cosine_distances",
    "linear_kernel", "polynomial_kernel", "sigmoid_kernel", "rbf_kernel", "laplacian_kernel",
    "cosine_similarity", "additive_chi2_kernel", "chi2_kernel",
    # scipy
    "directed_hausdorff_distances", "minkowski_distances", "wminkowski_distances",
    "sqeuclidean_distances", "correlation_distances", "hamming_distances", "jaccard_distances",
    "kulsinski_distances", "kulczynski1_distances", "seuclidean_distances",
    "cityblock_distances", "mahalanobis_distances", "chebyshev_distances",
    "braycurtis_distances", "canberra_distances", "jensenshannon_distances", "yule_distances",
    "dice_distances", "rogerstanimoto_distances", "russellrao_distances",
    "sokalmichener_distances", "sokalsneath_distances",
    # others
    "snr_distances",
    # aliases (linf is registered in C++ by the reference but not bound in its Python package;
    # it is bound here)
    "l1_distances", "l2_distances", "lp_distances", "linf_distances",
]
_CPDIST = ["cdist", "pdist", "k_neighbors_mask", "radius_neighbors_mask"]
_INTERNALS = [
    "pwand", "pwor", "pwxor", "pweq", "pwne", "pwlt", "pwgt", "pwle", "pwge",
    "pwand_sum", "pwor_sum", "pwxor_sum", "pweq_sum", "pwne_sum", "pweq_mean", "pwne_mean",
    "prf_div", "prf_ldiv", "prf_div_", "prf_ldiv_",
]

for _name in _METRICS + _CPDIST + _INTERNALS:
    globals()[_name] = getattr(torch.ops.torchpairwise, _name)

__all__ = list(_METRICS) + list(_CPDIST) + list(_INTERNALS)
