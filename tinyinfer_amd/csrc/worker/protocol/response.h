// Protocol v3 responses (interface of miniprefix/apps/protocol/response.h):
// each writes one line; `ready` also flushes.
#pragma once
#include "miniprefix/engine.h"

#include <ostream>
#include <string>
#include <vector>

namespace miniprefix::protocol {

void ready(std::ostream&, int vocabulary, int eos, int context, const std::string& backend);
void ok(std::ostream&);
void count(std::ostream&, std::size_t);
void logits(std::ostream&, const std::vector<float>&);
void events(std::ostream&, const std::vector<GenerationEvent>&);
void cost_stats(std::ostream&, const CostStats&);
void stats(std::ostream&, const RunnerStats&);
void step_stats(std::ostream&, const EngineStepStats&);
void error(std::ostream&, const std::string&);

}  // namespace miniprefix::protocol
