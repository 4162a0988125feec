// Test infrastructure: a C entry point over the reference's own header-only sampler
// (native/vulkan_decode/sampler.hpp, included from the reference tree by oracle/build_ref.sh), so the oracle's
// filtered distribution can be compared with Sampler::distribution on the same logits.
#include <cstdint>
#include <vector>
#include "sampler.hpp"

extern "C" int ref_distribution(const float *logits, int64_t n, float temperature, int top_k, float top_p,
                                int *ids_out, double *probs_out, int64_t cap) {
    SamplerParams p;
    p.temperature = temperature; p.top_k = top_k; p.top_p = top_p; p.seed = 1;
    Sampler s(p);
    std::vector<int> ids;
    std::vector<double> probs;
    s.distribution(logits, (size_t)n, ids, probs);
    if ((int64_t)ids.size() > cap) return -1;
    for (size_t i = 0; i < ids.size(); ++i) { ids_out[i] = ids[i]; probs_out[i] = probs[i]; }
    return (int)ids.size();
}
