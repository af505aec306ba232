// Persistent bit-packed boolean rows and the boolean count metrics over them.
//
//   _pack_bool(x) -> (words, popcounts)
//       bool rows [(B,) N, D] -> int32 words [(B,) N, W] (W = tpw_packed_words(D); bit k of a row
//       is bit k % 32 of word k / 32; padding bits zero) and int32 row popcounts [(B,) N].
//   _packed_bool_metric(words1, popcounts1, words2, popcounts2, d, metric) -> float32 [(B,) N, M]
//       one pass over packed rows for the boolean count metrics (hamming, jaccard, dice,
//       kulczynski1, kulsinski, rogerstanimoto, russellrao, sokalmichener, sokalsneath, yule)
//       and the reference's pw reductions (pw{and,or,xor,eq,ne}_sum, pw{eq,ne}_mean).
//
// A caller that packs once reuses the words across calls.  The packed kernel counts a & b per
// pair once and derives every other count from the row popcounts (xor = pa + pb - 2 and, ...),
// so each metric is one pass instead of the reference's 2-4 pw*_sum passes plus elementwise
// passes (pairwise_metrics.cpp:206-243,339-399).  The public boolean metrics on GPU bool
// tensors (bool_count_metric below) take the same counts and epilogue from the int8 matrix
// cores, straight from the bool bytes.  Results equal the reference's: each count is the
// float32 accumulator of ones the pw*_sum ops produce (exact below 2^24, then 2^24) and the
// float operations follow each composite in order, one rounding each.  russellrao's final
// "/ d" is a true division on the CPU and a multiply by fl(1 / d) on the GPU, as ATen divides
// a tensor by a CPU scalar on each device.
#include "tpw_common.h"

#include <ATen/Parallel.h>

#include <cstring>

namespace tpw_ext {
namespace {

constexpr int64_t kExact = int64_t(1) << 24;  // a float accumulator of ones stops here

struct MetricName {
    const char *name;
    int bmet;  // TPW_BMET_* or -1 for a pw reduction
    int op, red;
};

constexpr MetricName kMetrics[] = {
    {"hamming", TPW_BMET_HAMMING, 0, 0},
    {"jaccard", TPW_BMET_JACCARD, 0, 0},
    {"dice", TPW_BMET_DICE, 0, 0},
    {"kulczynski1", TPW_BMET_KULCZYNSKI1, 0, 0},
    {"kulsinski", TPW_BMET_KULSINSKI, 0, 0},
    {"rogerstanimoto", TPW_BMET_ROGERSTANIMOTO, 0, 0},
    {"russellrao", TPW_BMET_RUSSELLRAO, 0, 0},
    {"sokalmichener", TPW_BMET_SOKALMICHENER, 0, 0},
    {"sokalsneath", TPW_BMET_SOKALSNEATH, 0, 0},
    {"yule", TPW_BMET_YULE, 0, 0},
    // the reference's pw reductions (pairwise_binary.cpp:91-134)
    {"pwand_sum", -1, TPW_BIT_AND, TPW_RED_SUM},
    {"pwor_sum", -1, TPW_BIT_OR, TPW_RED_SUM},
    {"pwxor_sum", -1, TPW_BIT_XOR, TPW_RED_SUM},
    {"pweq_sum", -1, TPW_BIT_EQ, TPW_RED_SUM},
    {"pwne_sum", -1, TPW_BIT_NE, TPW_RED_SUM},
    {"pweq_mean", -1, TPW_BIT_EQ, TPW_RED_MEAN},
    {"pwne_mean", -1, TPW_BIT_NE, TPW_RED_MEAN},
};

const MetricName &metric_of(c10::string_view metric) {
    for (const auto &m : kMetrics)
        if (metric == m.name) return m;
    std::string names;
    for (const auto &m : kMetrics) names += std::string(names.empty() ? "" : ", ") + m.name;
    TORCH_CHECK(false, "_packed_bool_metric: unknown metric ", std::string(metric), ". Supported: ",
                names);
}

// ------------------------------------------------------------------ shapes
std::pair<at::Tensor, at::Tensor> check_pack_input(const at::Tensor &x) {
    TORCH_CHECK(x.scalar_type() == at::kBool, "_pack_bool: expected a bool tensor, got ",
                x.scalar_type());
    TORCH_CHECK(x.dim() == 2 || x.dim() == 3, "_pack_bool: expected [N, D] or [B, N, D] rows, got ",
                x.dim(), "-D");
    TORCH_CHECK(x.size(-1) >= 1, "_pack_bool: rows need at least one feature");
    auto x3 = as3(x);
    auto lead = x.sizes().vec();
    lead.pop_back();
    auto wshape = lead;
    wshape.push_back(tpw_packed_words(x.size(-1)));
    return {x3, at::empty(wshape, x.options().dtype(at::kInt))};
}

struct Packed3 {
    at::Tensor w1, p1, w2, p2;
    int64_t B, n, m, W;
    bool unbatched;
};

Packed3 check_packed(const at::Tensor &w1, const at::Tensor &p1, const at::Tensor &w2,
                     const at::Tensor &p2, int64_t d) {
    TORCH_CHECK(d >= 1, "_packed_bool_metric: d must be positive, got ", d);
    const int64_t W = tpw_packed_words(d);
    for (const at::Tensor *t : {&w1, &p1, &w2, &p2})
        TORCH_CHECK(t->scalar_type() == at::kInt, "_packed_bool_metric: packed words and popcounts "
                    "are int32 tensors (from _pack_bool), got ", t->scalar_type());
    TORCH_CHECK(w1.dim() == w2.dim() && (w1.dim() == 2 || w1.dim() == 3),
                "_packed_bool_metric: words must both be [N, W] or [B, N, W]");
    TORCH_CHECK(w1.size(-1) == W && w2.size(-1) == W, "_packed_bool_metric: ", W,
                " words per row expected for d = ", d, ", got ", w1.size(-1), " and ", w2.size(-1));
    const bool ub = w1.dim() == 2;
    TORCH_CHECK(ub || w1.size(0) == w2.size(0), "_packed_bool_metric: batch sizes do not match");
    TORCH_CHECK(p1.dim() == w1.dim() - 1 && p2.dim() == w2.dim() - 1 &&
                    p1.sizes() == w1.sizes().slice(0, w1.dim() - 1) &&
                    p2.sizes() == w2.sizes().slice(0, w2.dim() - 1),
                "_packed_bool_metric: popcounts must have one entry per packed row");
    TORCH_CHECK(w1.device() == w2.device() && w1.device() == p1.device() && w1.device() == p2.device(),
                "_packed_bool_metric: all tensors must be on one device");
    Packed3 r;
    r.w1 = as3(w1);
    r.w2 = as3(w2);
    r.p1 = (ub ? p1.unsqueeze(0) : p1).contiguous();
    r.p2 = (ub ? p2.unsqueeze(0) : p2).contiguous();
    r.B = r.w1.size(0);
    r.n = r.w1.size(1);
    r.m = r.w2.size(1);
    r.W = W;
    r.unbatched = ub;
    return r;
}

inline float sat(int64_t c) { return (float)(c < kExact ? c : kExact); }

// ------------------------------------------------------------------ CPU
std::tuple<at::Tensor, at::Tensor> pack_bool_cpu(const at::Tensor &x) {
    auto xw = check_pack_input(x);
    const at::Tensor &x3 = xw.first;
    at::Tensor words = xw.second;
    const int64_t rows = x3.size(0) * x3.size(1), d = x3.size(2), W = words.size(-1);
    auto lead = x.sizes().vec();
    lead.pop_back();
    at::Tensor pops = at::empty(lead, x.options().dtype(at::kInt));
    const bool *src = x3.data_ptr<bool>();
    uint32_t *dst = reinterpret_cast<uint32_t *>(words.data_ptr<int32_t>());
    int32_t *pc = pops.data_ptr<int32_t>();
    at::parallel_for(0, rows, 64, [&](int64_t lo, int64_t hi) {
        for (int64_t r = lo; r < hi; ++r) {
            uint32_t *w = dst + r * W;
            std::memset(w, 0, sizeof(uint32_t) * W);
            const bool *p = src + r * d;
            for (int64_t k = 0; k < d; ++k)
                if (p[k]) w[k >> 5] |= 1u << (k & 31);
            int64_t c = 0;
            for (int64_t q = 0; q < W; ++q) c += __builtin_popcount(w[q]);
            pc[r] = (int32_t)c;
        }
    });
    return {words, pops};
}

float count_metric_cpu(int bmet, int64_t n11, int64_t pa, int64_t pb, int64_t d) {
    const int64_t x = pa + pb - 2 * n11;
    const float A = sat(n11), S = sat(x), df = (float)d;
    switch (bmet) {
        case TPW_BMET_HAMMING: return S / df;
        case TPW_BMET_JACCARD: {
            const float O = sat(pa + pb - n11);
            return O != 0.0f ? S / O : 0.0f;
        }
        case TPW_BMET_DICE: return S / (2.0f * A + S);
        case TPW_BMET_KULCZYNSKI1: return A / S;
        case TPW_BMET_KULSINSKI: {
            const float num = (S - A) + df, den = S + df;
            return num / den;
        }
        case TPW_BMET_ROGERSTANIMOTO:
        case TPW_BMET_SOKALMICHENER: {
            const float R = 2.0f * S, E = sat(d - x);
            return R / (E + R);
        }
        case TPW_BMET_RUSSELLRAO: return (df - A) / df;
        case TPW_BMET_SOKALSNEATH: {
            const float R = 2.0f * S;
            return R / (A + R);
        }
        default: {  // yule
            const float n10 = sat(pa - n11), n01 = sat(pb - n11), n00 = sat(d - pa - pb + n11);
            const float hR = n10 * n01, num = 2.0f * hR, prod = A * n00, den = prod + hR;
            return den != 0.0f ? num / den : 0.0f;
        }
    }
}

at::Tensor packed_bool_metric_cpu(const at::Tensor &w1, const at::Tensor &p1, const at::Tensor &w2,
                                  const at::Tensor &p2, int64_t d, c10::string_view metric) {
    const MetricName &mt = metric_of(metric);
    Packed3 t = check_packed(w1, p1, w2, p2, d);
    auto out = at::empty({t.B, t.n, t.m}, t.w1.options().dtype(at::kFloat));
    const uint32_t *a = reinterpret_cast<const uint32_t *>(t.w1.data_ptr<int32_t>());
    const uint32_t *b = reinterpret_cast<const uint32_t *>(t.w2.data_ptr<int32_t>());
    const int32_t *pa = t.p1.data_ptr<int32_t>(), *pb = t.p2.data_ptr<int32_t>();
    float *o = out.data_ptr<float>();
    const int64_t W = t.W, n = t.n, m = t.m;
    at::parallel_for(0, t.B * n, 1, [&](int64_t lo, int64_t hi) {
        for (int64_t r = lo; r < hi; ++r) {
            const int64_t bb = r / n;
            const uint32_t *ar = a + r * W;
            for (int64_t j = 0; j < m; ++j) {
                const uint32_t *br = b + (bb * m + j) * W;
                int64_t c = 0;
                for (int64_t q = 0; q < W; ++q) {
                    uint32_t v;
                    switch (mt.op) {
                        case TPW_BIT_OR: v = ar[q] | br[q]; break;
                        case TPW_BIT_AND: v = ar[q] & br[q]; break;
                        default: v = ar[q] ^ br[q];  // xor, ne, eq (d - ne)
                    }
                    c += __builtin_popcount(v);
                }
                float val;
                if (mt.bmet >= 0) {
                    val = count_metric_cpu(mt.bmet, c, pa[r], pb[bb * m + j], d);
                } else {
                    if (mt.op == TPW_BIT_EQ) c = d - c;
                    val = sat(c);
                    if (mt.red == TPW_RED_MEAN) val = val / (float)d;
                }
                o[r * m + j] = val;
            }
        }
    });
    return t.unbatched ? out.squeeze(0) : out;
}

// ------------------------------------------------------------------ GPU
std::tuple<at::Tensor, at::Tensor> pack_bool_cuda(const at::Tensor &x) {
    auto xw = check_pack_input(x);
    DeviceGuard guard(x.device());
    const at::Tensor &x3 = xw.first;
    at::Tensor words = xw.second;
    auto lead = x.sizes().vec();
    lead.pop_back();
    at::Tensor pops = at::empty(lead, x.options().dtype(at::kInt));
    check_rc(tpw_pack_bool_rows(reinterpret_cast<const uint8_t *>(x3.data_ptr<bool>()),
                                x3.size(0) * x3.size(1), x3.size(2),
                                reinterpret_cast<uint32_t *>(words.data_ptr<int32_t>()),
                                pops.data_ptr<int32_t>(), current_stream()),
             "_pack_bool");
    return {words, pops};
}

at::Tensor packed_bool_metric_cuda(const at::Tensor &w1, const at::Tensor &p1, const at::Tensor &w2,
                                   const at::Tensor &p2, int64_t d, c10::string_view metric) {
    const MetricName &mt = metric_of(metric);
    Packed3 t = check_packed(w1, p1, w2, p2, d);
    DeviceGuard guard(w1.device());
    auto out = at::empty({t.B, t.n, t.m}, t.w1.options().dtype(at::kFloat));
    if (t.B * t.n * t.m > 0) {
        const uint32_t *a = reinterpret_cast<const uint32_t *>(t.w1.data_ptr<int32_t>());
        const uint32_t *b = reinterpret_cast<const uint32_t *>(t.w2.data_ptr<int32_t>());
        if (mt.bmet >= 0)
            check_rc(tpw_bool_count_metric(a, b, t.p1.data_ptr<int32_t>(), t.p2.data_ptr<int32_t>(), t.B,
                                           t.n, t.m, d, mt.bmet, out.data_ptr<float>(), current_stream()),
                     "_packed_bool_metric");
        else
            check_rc(tpw_bool_pairwise_reduce_counted(a, b, t.p1.data_ptr<int32_t>(), t.p2.data_ptr<int32_t>(), t.B,
                                                      t.n, t.m, d, mt.op, mt.red, out.data_ptr<float>(),
                                                      current_stream()),
                     "_packed_bool_metric");
    }
    return t.unbatched ? out.squeeze(0) : out;
}

template <typename Sig>
c10::TypedOperatorHandle<Sig> op_handle(const char *name) {
    return c10::Dispatcher::singleton().findSchemaOrThrow(name, "").typed<Sig>();
}

}  // namespace

std::tuple<at::Tensor, at::Tensor> pack_bool(const at::Tensor &x) {
    static auto op = op_handle<std::tuple<at::Tensor, at::Tensor>(const at::Tensor &)>("torchpairwise::_pack_bool");
    return op.call(x);
}

at::Tensor packed_bool_metric(const at::Tensor &w1, const at::Tensor &p1, const at::Tensor &w2,
                              const at::Tensor &p2, int64_t d, c10::string_view metric) {
    static auto op = op_handle<at::Tensor(const at::Tensor &, const at::Tensor &, const at::Tensor &,
                                          const at::Tensor &, int64_t, c10::string_view)>(
        "torchpairwise::_packed_bool_metric");
    return op.call(w1, p1, w2, p2, d, metric);
}

at::Tensor bool_count_metric(const at::Tensor &x1, const at::Tensor &x2, c10::string_view metric) {
    // GPU bool rows of the public metrics: one pass on the int8 matrix cores straight from the
    // bytes (the AND count of two 0/1 rows is their int8 dot product); other inputs, shapes the
    // composites reject and empty rows take the reference's composite
    if (!x1.is_cuda() || !x2.is_cuda() || x1.scalar_type() != at::kBool || x2.scalar_type() != at::kBool ||
        x1.dim() != x2.dim() || (x1.dim() != 2 && x1.dim() != 3) || x1.size(-1) < 1 ||
        x1.size(-1) != x2.size(-1) || (x1.dim() == 3 && x1.size(0) != x2.size(0)) ||
        x1.device() != x2.device())
        return at::Tensor();
    const MetricName &mt = metric_of(metric);
    DeviceGuard guard(x1.device());
    const bool unbatched = x1.dim() == 2;
    auto a = (unbatched ? x1.unsqueeze(0) : x1).contiguous();
    auto b = x2.is_same(x1) ? a : (unbatched ? x2.unsqueeze(0) : x2).contiguous();
    auto out = at::empty({a.size(0), a.size(1), b.size(1)}, a.options().dtype(at::kFloat));
    if (out.numel() > 0) bool_bytes_cuda(a, b, mt.bmet, mt.op, mt.red, out);
    return unbatched ? out.squeeze(0) : out;
}

TORCH_LIBRARY_FRAGMENT(torchpairwise, m) {
    m.def("_pack_bool(Tensor x) -> (Tensor words, Tensor popcounts)");
    m.def("_packed_bool_metric(Tensor words1, Tensor popcounts1, Tensor words2, Tensor popcounts2, "
          "int d, str metric) -> Tensor");
}

TORCH_LIBRARY_IMPL(torchpairwise, CPU, m) {
    m.impl("_pack_bool", TORCH_FN(pack_bool_cpu));
    m.impl("_packed_bool_metric", TORCH_FN(packed_bool_metric_cpu));
}

TORCH_LIBRARY_IMPL(torchpairwise, CUDA, m) {
    m.impl("_pack_bool", TORCH_FN(pack_bool_cuda));
    m.impl("_packed_bool_metric", TORCH_FN(packed_bool_metric_cuda));
}

}  // namespace tpw_ext
