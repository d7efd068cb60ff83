// TEST INFRASTRUCTURE ONLY.  A C-ABI shim over the reference's own CPU truth
// (cpp/reference/qwen35.cpp, compiled from /root/reference by oracle/Makefile
// into oracle/_ref/).  It exists so tests can check the C restatement in
// oracle.c against the compiled reference on identical inputs; the product
// never loads it.
#include "reference/qwen35.hpp"

#include <cstddef>
#include <exception>
#include <span>

using namespace raftinfer::reference;

extern "C" {

// qwen35.hpp:82-85 / qwen35.cpp:254-382
int ref_gated_full_attention(const float *input, const float *qnw,
                             const float *knw, const float *ow, float *output,
                             std::size_t tokens, std::size_t hidden,
                             std::size_t hq, std::size_t hkv, std::size_t d,
                             std::size_t rotary_dim, std::size_t position,
                             float rope_base, float eps) {
  try {
    const FullAttentionReferenceArgs args{tokens, hidden, hq, hkv, d,
                                          rotary_dim, position, rope_base, eps};
    const std::size_t stride = hq * d + 2 * hkv * d + hidden;
    qwen35_gated_full_attention(
        std::span<const float>(input, tokens * stride),
        std::span<float>(output, tokens * hidden),
        FullAttentionReferenceWeights{std::span<const float>(qnw, d),
                                      std::span<const float>(knw, d),
                                      std::span<const float>(ow, hidden * hidden)},
        args);
    return 0;
  } catch (const std::exception &) {
    return -1;
  }
}

// qwen35.hpp:97-101 / qwen35.cpp:528-549
int ref_gated_delta_prefill(const float *input, const float *conv_weight,
                            const float *recurrent_a, const float *dt_bias,
                            const float *norm_w, float *output,
                            float *conv_state, float *rec_state,
                            std::size_t tokens, std::size_t hidden,
                            std::size_t hk, std::size_t hv, std::size_t dk,
                            std::size_t dv, std::size_t width, float eps) {
  try {
    const GatedDeltaReferenceArgs args{tokens, hidden, hk, hv, dk, dv, width, eps};
    GatedDeltaReferenceState state(args);
    const std::size_t conv_dim = 2 * hk * dk + hv * dv;
    const std::size_t stride = conv_dim + 2 * hv + hidden;
    std::copy(conv_state, conv_state + state.convolution.size(),
              state.convolution.begin());
    std::copy(rec_state, rec_state + state.recurrent.size(),
              state.recurrent.begin());
    qwen35_gated_delta_prefill(
        std::span<const float>(input, tokens * stride),
        std::span<float>(output, tokens * hidden),
        GatedDeltaReferenceWeights{std::span<const float>(conv_weight, conv_dim * width),
                                   std::span<const float>(recurrent_a, hv),
                                   std::span<const float>(dt_bias, hv),
                                   std::span<const float>(norm_w, dv)},
        args, state);
    std::copy(state.convolution.begin(), state.convolution.end(), conv_state);
    std::copy(state.recurrent.begin(), state.recurrent.end(), rec_state);
    return 0;
  } catch (const std::exception &) {
    return -1;
  }
}

} // extern "C"
