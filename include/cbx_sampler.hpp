// cbx_sampler.hpp -- header-only C++ front end with the reference's signature.
//
//   int32_t sample_next_token_ex(const std::vector<float>& logits,
//                                const std::vector<int32_t>& generated,
//                                const chatterbox_sampling_params& params,
//                                std::mt19937& rng);
//
// is tts_cpp::chatterbox::detail::sample_next_token_ex (src/main.cpp:726-801,
// declared at src/chatterbox_t3_internal.h:144-148).  Here it runs on the GPU
// through the C ABI (cbx_sampler.h) and returns the reference's token:
//
// * The uniform is what the reference's std::discrete_distribution takes from
//   `rng`: std::generate_canonical<double, 53> over two 32-bit outputs
//   (libstdc++ random.tcc:3348-3375), read from a copy of the engine.
// * The caller's engine advances by those two outputs only when the reference
//   would have drawn (CBX_INFO_DREW): not for temp <= 0, an all -inf row, or a
//   vocabulary of one.
//
// A Sampler owns one handle (its stream and staging buffers); like the
// reference engine it is not thread-safe, so use one per decode thread.  The
// free function keeps one Sampler per thread on device 0.
#pragma once

#include <cstdint>
#include <limits>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "cbx_sampler.h"

namespace cbx {

// Field for field chatterbox_sampling_params (chatterbox_t3_internal.h:113-118).
struct chatterbox_sampling_params {
    int32_t top_k = 1000;
    float top_p = 0.95f;
    float temp = 0.8f;
    float repeat_penalty = 1.2f;
};

// The uniform std::discrete_distribution would draw from `rng`, without
// advancing it.
inline double peek_uniform(const std::mt19937& rng) {
    std::mt19937 copy = rng;
    return std::generate_canonical<double, std::numeric_limits<double>::digits>(copy);
}

class Sampler {
public:
    explicit Sampler(int32_t device = 0, int32_t max_vocab = 32768, int32_t max_history = 1 << 16) {
        if (cbx_sampler_create(&h_, device, max_vocab, max_history) != CBX_OK)
            throw std::runtime_error(std::string("cbx_sampler_create: ") + cbx_last_error());
    }
    ~Sampler() { cbx_sampler_destroy(h_); }
    Sampler(const Sampler&) = delete;
    Sampler& operator=(const Sampler&) = delete;

    cbx_sampler* handle() const { return h_; }

    int32_t sample_next_token_ex(const std::vector<float>& logits,
                                 const std::vector<int32_t>& generated,
                                 const chatterbox_sampling_params& params, std::mt19937& rng) {
        const cbx_params p{params.top_k, params.top_p, params.temp, params.repeat_penalty, 0.0f,
                           0.0f};
        int32_t token = 0;
        uint32_t info = 0;
        const int rc = cbx_sample_row(h_, logits.data(), (int32_t)logits.size(),
                                      generated.empty() ? nullptr : generated.data(),
                                      (int32_t)generated.size(), &p, peek_uniform(rng), &token,
                                      &info);
        if (rc != CBX_OK) throw std::runtime_error(std::string("cbx_sample_row: ") + cbx_last_error());
        if (info & CBX_INFO_DREW) rng.discard(2);
        return token;
    }

private:
    cbx_sampler* h_ = nullptr;
};

inline int32_t sample_next_token_ex(const std::vector<float>& logits,
                                    const std::vector<int32_t>& generated,
                                    const chatterbox_sampling_params& params, std::mt19937& rng) {
    thread_local Sampler sampler;
    return sampler.sample_next_token_ex(logits, generated, params, rng);
}

}  // namespace cbx
