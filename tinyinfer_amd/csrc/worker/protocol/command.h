// Protocol v3 commands (interface of miniprefix/apps/protocol/command.h:1-8):
// one text line per command; fields are whitespace separated, extra
// trailing fields are ignored, integers are read as formatted stream
// extraction ("+1" and "1x" both read 1), and the validation order of the
// reference is kept, so that a client sees the same errors.
#pragma once
#include "miniprefix/request.h"

#include <string>
#include <vector>

namespace miniprefix::protocol {

enum class Kind { Submit, Step, StepStats, Cancel, ClearPrefix, Cache, Reuse, Forward, Release, Stats, CostStats, CostTiming, Quit };

struct Command {
    Kind kind;
    int id = 0;                  // request or diagnostic sequence id, timing flag
    Request request;             // SUBMIT
    std::vector<TokenId> input;  // FORWARD, REUSE
};

// Throws std::invalid_argument with the protocol's error text.
Command parse(const std::string& line);

}  // namespace miniprefix::protocol
