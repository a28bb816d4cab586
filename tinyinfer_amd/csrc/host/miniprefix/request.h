// Value contracts of a generation request (reference:
// miniprefix/include/miniprefix/request.h:12-36). Same names and meaning.
#pragma once
#include <cstdint>
#include <optional>
#include <string>
#include <vector>

namespace miniprefix {

using TokenId = std::int32_t;
using RequestId = std::string;

enum class FinishReason { Eos, Length, Cancelled, Error };

struct GenerationOptions {
    std::uint32_t max_new_tokens = 32;
    std::optional<TokenId> eos_token_id;
};

struct Request {
    RequestId id;
    std::vector<TokenId> prompt_token_ids;
    GenerationOptions generation;
};

// A committed output token is delivered exactly once; a finish-only event
// carries no token.
struct GenerationEvent {
    RequestId request_id;
    std::optional<TokenId> token_id;
    std::optional<FinishReason> finish_reason;
    std::string error_message;
};

}  // namespace miniprefix
