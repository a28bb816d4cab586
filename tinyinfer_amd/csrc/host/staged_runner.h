// Cross-request batching: an optional interface a ModelRunner may also
// implement. It has no counterpart in the reference, whose Engine calls
// ModelRunner::append once per request (miniprefix/src/engine/engine.cpp:81-90).
// This header depends only on the reference's value contracts, so a runner
// implementing it builds inside the reference tree as well as here.
#pragma once
#include "miniprefix/request.h"

#include <vector>

namespace miniprefix {

struct StagedResult {
    TokenId argmax = 0;  // first index of the last row's maximum logit (std::max_element)
    bool finite = true;  // every logit of every row of the item finite
};

// stage() performs an append's KV transaction (reservation, copy-on-write,
// commit) at once, in call order, and queues its forward; run_staged()
// computes every queued forward in one device pass and returns one result
// per staged item, in order. Metadata commits before compute, so a
// non-finite result cannot be rolled back: callers treat it as fatal.
//
// Within one pass the queued forwards run concurrently: none may read a
// page another queued forward writes. A caller that maps cached pages into
// a new sequence while forwards are queued asks shares_staged_pages() and
// runs the queue first when it answers true.
class StagedRunner {
public:
    virtual ~StagedRunner() = default;
    virtual void stage(const RequestId& id, const std::vector<TokenId>& tokens) = 0;
    virtual std::vector<StagedResult> run_staged() = 0;
    virtual void discard_staged() noexcept = 0;
    // True when sequence `id` references a block that a queued forward writes.
    virtual bool shares_staged_pages(const RequestId& id) const = 0;
    // True when staging `tokens` more for sequence `id` would take pages
    // from the pool (new pages or a copy-on-write target) or, with
    // `publishes`, publish into a prefix cache, whose evictions return pages
    // to the pool. A caller whose queued items may release their sequences
    // once their results are known runs the queue before such a stage, so
    // that the pool sees the releases first.
    virtual bool stage_touches_pool(const RequestId& id, std::size_t tokens, bool publishes) const = 0;
};

}  // namespace miniprefix
