// The engine's decode loop (chatterbox_engine.cpp:326-353) written against the
// header-only front end include/cbx_sampler.hpp, next to the same loop driven
// by the CPU oracle (std::discrete_distribution on the same std::mt19937
// seed).  Prints "OK <steps>" when every token matches, else the first
// mismatch.  usage: shim_engine_loop <steps> <seed>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

#include "../../include/cbx_sampler.hpp"
#include "../../oracle/cbx_oracle.h"

int main(int argc, char** argv) {
    const int steps = argc > 1 ? atoi(argv[1]) : 300;
    const uint32_t seed = argc > 2 ? (uint32_t)strtoul(argv[2], nullptr, 0) : 42u;
    const int V = 6563;
    std::mt19937 gen(20261201u);
    std::normal_distribution<float> nd(0.0f, 3.0f);
    std::vector<float> all((size_t)steps * V);
    for (auto& x : all) x = nd(gen);
    for (int t = 0; t < steps; ++t)
        for (int k = 0; k < 5; ++k) all[(size_t)t * V + (gen() % V)] = 12.0f;

    cbx::chatterbox_sampling_params sp;  // reference defaults 1000, 0.95, 0.8, 1.2
    cbx_oracle_params op{sp.top_k, sp.top_p, sp.temp, sp.repeat_penalty, 0.0f, 0.0f};
    std::vector<int32_t> ref(steps);
    cbx_oracle_run_mt19937(all.data(), steps, V, nullptr, 0, 1, &op, seed, ref.data(), nullptr);

    std::mt19937 rng(seed);
    std::vector<int32_t> generated;
    std::vector<float> logits(V);
    for (int t = 0; t < steps; ++t) {
        logits.assign(all.begin() + (size_t)t * V, all.begin() + (size_t)(t + 1) * V);
        const int32_t tok = cbx::sample_next_token_ex(logits, generated, sp, rng);
        if (tok != ref[t]) {
            printf("MISMATCH step %d gpu %d ref %d\n", t, tok, ref[t]);
            return 1;
        }
        generated.push_back(tok);
    }
    // greedy: no draws, the engine must not advance
    std::mt19937 a(seed), b(seed);
    cbx::chatterbox_sampling_params g = sp;
    g.temp = 0.0f;
    logits.assign(all.begin(), all.begin() + V);
    (void)cbx::sample_next_token_ex(logits, generated, g, a);
    if (a != b) {
        printf("MISMATCH greedy call advanced the engine\n");
        return 1;
    }
    printf("OK %d\n", steps);
    return 0;
}
