// MiniPrefix worker over the HIP runner: the reference worker's command line
// and protocol v3 on stdin/stdout (miniprefix/apps/worker.cpp:6-21), with the
// backends of this worker:
//   hip       the HIP runner in the exact arithmetic (logits bit-identical
//             to the reference CPU runner), the drop-in for cpu/cuda;
//   hip-fast  the HIP runner in the fast arithmetic (FP32 matrix cores,
//             flash-decoding attention; logits within 1e-3 relative).
// usage: miniprefix_worker MODEL hip|hip-fast CONTEXT [BATCH TOKENS CHUNK BLOCK_TOKENS KV_BLOCKS PREFIX_BLOCKS]
// MODEL is an MPFX0001 checkpoint. Start-up errors go to stderr with exit
// status 1; after the READY line every error is an ERROR response.
#include "mp_hip.h"
#include "miniprefix/engine.h"
#include "protocol/response.h"
#include "protocol/session.h"

#include <iostream>
#include <stdexcept>
#include <string>

using namespace miniprefix;

namespace {

constexpr const char* kUsage =
    "usage: miniprefix_worker MODEL hip|hip-fast CONTEXT [BATCH TOKENS CHUNK BLOCK_TOKENS KV_BLOCKS PREFIX_BLOCKS]";

std::unique_ptr<ModelRunner> runner_for(const std::string& backend, std::shared_ptr<ModelWeights> weights,
                                        int context, KvCacheConfig kv) {
    if (backend == "hip") return make_hip_runner(std::move(weights), context, kv);
    if (backend == "hip-fast") return make_hip_runner(std::move(weights), context, kv, MP_ARITHMETIC_FAST);
    throw std::invalid_argument("backend unavailable in this build");
}

}  // namespace

int main(int argc, char** argv) {
    try {
        if (argc < 4 || argc > 10) throw std::invalid_argument(kUsage);
        auto arg = [&](int i) { return std::stoi(argv[i]); };
        const auto weights = ModelWeights::load(argv[1]);
        const std::string backend = argv[2];
        const int context = arg(3);
        KvCacheConfig kv;
        if (argc > 7) kv.block_tokens = arg(7);
        if (argc > 8) kv.max_blocks = arg(8);
        if (argc > 9) kv.prefix_cache_blocks = arg(9);
        EngineConfig config;
        config.context = context;
        if (argc > 4) config.max_batch_size = arg(4);
        if (argc > 5) config.token_budget = arg(5);
        if (argc > 6) config.prefill_chunk = arg(6);
        Engine engine(runner_for(backend, weights, context, kv), config);
        protocol::ready(std::cout, weights->config.vocabulary, weights->config.eos, context, backend);
        return protocol::serve(engine, std::cin, std::cout);
    } catch (const std::exception& e) {
        std::cerr << e.what() << '\n';
        return 1;
    }
}
