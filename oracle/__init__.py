"""CPU oracle for the torchpairwise hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import this package, and only as the checker (or the timed CPU baseline), never as the
product path: the product (``torchpairwise_amd``) fails loudly when its HIP library is
missing and never routes through here.

Contents (each function cites the reference file:line it restates):

* ``oracle.pairwise`` — numpy / torch restatements:
  - boolean metrics (hamming, jaccard, pw*_sum / pw*_mean) as integer popcounts followed by
    the reference's float32 arithmetic (bit-exact);
  - the ATen-routed metrics (euclidean, manhattan, minkowski, chebyshev) as ``torch.cdist``
    + autograd on CPU, which *is* the reference's arithmetic (pairwise_metrics.cpp:24-49,
    160-168,299-306 call at::cdist);
  - cosine as the reference's torch-op composite with prf_div "identity";
  - directed Hausdorff as an fp32 brute force with per-operation rounding (no FMA) and the
    reference's tie rules, plus its backward scatter;
  - the neighbour masks: each row's k + 1 smallest by a stable sort, and dist <= epsilon;
  - the reference's VALU kernels (_ppminkowski, _wminkowski, _canberra, _braycurtis,
    _additive_chi2_kernel, _sqjensenshannon, _haversine, _snr, _sqmahalanobis) as
    differentiable torch broadcasts over [n, m, d].
* ``oracle/cref.c`` (built by ``oracle/Makefile`` into ``oracle/_build/liboracle_cref.so``,
  wrapped by ``oracle.cref``) — a C restatement of the reference's CPU loops: the
  sequential early-break Hausdorff loop and the one-output-per-iteration binary
  reduction, compiled with -ffp-contract=off like the reference's x86-64 build.  It pins
  the numpy brute force (same bits through a different algorithm) and is the timed CPU
  baseline ("port") in bench.py.

Pinning (what checks each function; see tests/test_oracle.py):
  hamming / jaccard / pw* : scipy.spatial.distance.cdist (float64 then float32 — double
      rounding of a quotient of integers < 2^24 is innocuous), closed forms (d a power of
      two gives exact dyadics, all-zero rows give jaccard 0), brute force per element, the
      C restatement, committed golden vectors.
  cdist-routed metrics    : scipy.spatial.distance.cdist in float64, autograd.gradcheck.
  cosine                  : sklearn.metrics.pairwise.cosine_distances, gradcheck in float64.
  directed Hausdorff      : the C early-break restatement (bit-exact value and indices),
      scipy.spatial.distance.directed_hausdorff (value), hand-built tie cases, gradcheck.
  VALU family             : scipy.spatial.distance.cdist fixtures (sqeuclidean, weighted
      minkowski p = 1, 2, 3, seuclidean, canberra with a 0 / 0 term, braycurtis),
      gradcheck in float64, closed forms (p = 0 fills d, p = 2 of pp = squared euclidean).
  chi2 / JS / haversine   : sklearn additive_chi2_kernel, chi2_kernel, haversine_distances and
      scipy jensenshannon (base e and 2) fixtures, gradcheck, closed forms (antipodes are
      pi apart, disjoint distributions give ln 2).
  snr                     : the variance ratio var(x2 - x1) / var(x1) in numpy, gradcheck.
  sqmahalanobis           : scipy cdist 'mahalanobis' fixture, VI = I gives sqeuclidean.
  neighbour masks         : sklearn.neighbors kneighbors_graph / radius_neighbors_graph
      (connectivity) on tie-free data, hand-built ties / NaN / -0 cases with hand-derived
      masks (golden vectors), and the selection properties (row count, every selected
      entry <= every unselected one).
"""
