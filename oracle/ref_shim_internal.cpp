// TEST INFRASTRUCTURE ONLY.  Compiles the reference's CPU truth
// (cpp/reference/qwen35.cpp, included from the reference tree at build time by
// oracle/Makefile) in this translation unit, so that its file-local helpers
// (RMSNorm, partial RoPE) can be exposed to the tests next to the public
// functions ref_shim.cpp wraps.  The product never loads it.
#include "reference/qwen35.cpp"

#include <cstddef>
#include <exception>
#include <span>

extern "C" {

// qwen35.cpp:297-312: per (token, head) vector, rms_norm_with_multiplier
// (weight base 0) then apply_partial_rope at position_offset + token.
int ref_qk_norm_rope(const float *input, const float *weight, float *output,
                     std::size_t tokens, std::size_t heads, std::size_t head_dim,
                     std::size_t rotary_dim, std::size_t position_offset,
                     float rope_base, float epsilon) {
  try {
    for (std::size_t t = 0; t < tokens; ++t)
      for (std::size_t h = 0; h < heads; ++h) {
        const std::size_t base = (t * heads + h) * head_dim;
        std::span<float> out(output + base, head_dim);
        raftinfer::reference::rms_norm_with_multiplier(
            std::span<const float>(input + base, head_dim),
            std::span<const float>(weight, head_dim), out, 1, head_dim, epsilon, 0.0F);
        raftinfer::reference::apply_partial_rope(out, rotary_dim, position_offset + t,
                                                 rope_base);
      }
    return 0;
  } catch (const std::exception &) {
    return -1;
  }
}

} // extern "C"
