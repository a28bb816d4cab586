// Protocol v3 of the worker (tinyinfer_amd/csrc/worker) against the wire
// format the reference pins in miniprefix/tests/worker_protocol_test.cpp:9-104:
// parse errors and their order, the exact response lines, a session
// transcript over a recording runner, end of input without QUIT, and the
// refusal of direct runner commands once the engine has failed. Built
// against this repository's protocol and host runtime and, where the
// reference tree exists, against the reference's own protocol sources.
#include "protocol/command.h"
#include "protocol/response.h"
#include "protocol/session.h"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <iostream>
#include <limits>
#include <map>
#include <sstream>

using namespace miniprefix;

namespace {

int failures = 0;
#define EXPECT(cond)                                                              \
    do {                                                                          \
        if (!(cond)) {                                                            \
            std::fprintf(stderr, "%s:%d: expected %s\n", __FILE__, __LINE__, #cond); \
            ++failures;                                                           \
        }                                                                         \
    } while (0)

std::string parse_error(const std::string& line) {
    try {
        protocol::parse(line);
    } catch (const std::invalid_argument& e) {
        return e.what();
    }
    return "";
}

void parse_errors_in_validation_order() {
    const std::pair<const char*, const char*> cases[] = {
        {"", "unknown command"},
        {"   ", "unknown command"},
        {"submit 1 1 -1 1 1", "unknown command"},
        {"STEPS", "unknown command"},
        {"SUBMIT", "missing integer"},
        {"SUBMIT 1 1 -1", "missing integer"},          // count missing before id/limit are judged
        {"SUBMIT 0 1 -1 1 1", "invalid request"},
        {"SUBMIT 1 0 -1 1 1", "invalid request"},
        {"SUBMIT 1 1 -1 0", "invalid token count"},
        {"SUBMIT 1 1 -1 131073", "invalid token count"},
        {"SUBMIT 1 1 -1 3 1 2", "missing integer"},
        {"SUBMIT 1 1 -5 1 4", "invalid EOS"},          // judged after the tokens
        {"SUBMIT 1 1 -5 1", "missing integer"},
        {"FORWARD 1", "missing integer"},
        {"FORWARD 1 0", "invalid token count"},
        {"FORWARD 0 2 1", "missing integer"},
        {"FORWARD 0 1 1", "invalid diagnostic sequence"},
        {"REUSE -3 1 1", "invalid diagnostic sequence"},
        {"CACHE x", "missing integer"},
        {"RELEASE", "missing integer"},
        {"CANCEL 99999999999", "missing integer"},    // does not fit an int
        {"COST_TIMING -1", "invalid timing flag"},
        {"COST_TIMING", "missing integer"},
    };
    for (const auto& c : cases) {
        const std::string got = parse_error(c.first);
        if (got != c.second) std::fprintf(stderr, "parse(\"%s\"): \"%s\", want \"%s\"\n", c.first, got.c_str(), c.second);
        EXPECT(got == c.second);
    }
}

void parse_accepts() {
    auto s = protocol::parse("\t SUBMIT 7 3 5 3 10 11 12 extra fields\r");
    EXPECT(s.kind == protocol::Kind::Submit && s.request.id == "7" && s.request.generation.max_new_tokens == 3);
    EXPECT(s.request.generation.eos_token_id && *s.request.generation.eos_token_id == 5);
    EXPECT((s.request.prompt_token_ids == std::vector<TokenId>{10, 11, 12}));
    auto n = protocol::parse("SUBMIT 8 1 -1 1 0");
    EXPECT(!n.request.generation.eos_token_id);
    auto f = protocol::parse("FORWARD 3 2 -4 +5");  // token values are the runner's to judge
    EXPECT(f.kind == protocol::Kind::Forward && f.id == 3 && (f.input == std::vector<TokenId>{-4, 5}));
    EXPECT(protocol::parse("REUSE 2 1 9").kind == protocol::Kind::Reuse);
    EXPECT(protocol::parse("CANCEL -7").id == -7 && protocol::parse("CACHE 12abc").id == 12);
    EXPECT(protocol::parse("COST_TIMING 0").kind == protocol::Kind::CostTiming);
    const std::pair<const char*, protocol::Kind> plain[] = {
        {"STEP", protocol::Kind::Step},           {"STEP_STATS x", protocol::Kind::StepStats},
        {"CLEAR_PREFIX", protocol::Kind::ClearPrefix}, {"COST_STATS", protocol::Kind::CostStats},
        {"STATS 1 2", protocol::Kind::Stats},     {"QUIT now", protocol::Kind::Quit}};
    for (const auto& p : plain) EXPECT(protocol::parse(p.first).kind == p.second);
    std::string big = "FORWARD 1 131072";
    for (int i = 0; i < 131072; ++i) big += " 1";
    EXPECT(protocol::parse(big).input.size() == 131072);
}

void response_lines() {
    std::ostringstream out;
    protocol::ready(out, 49152, 0, 2048, "hip");
    protocol::ok(out);
    protocol::count(out, 0);
    protocol::logits(out, {1.0F, -2.5e-8F, 3.14159274F, 65504.0F, std::numeric_limits<float>::infinity()});
    protocol::events(out, {{"r1", 7, FinishReason::Length, ""}, {"r2", std::nullopt, FinishReason::Cancelled, "x"}});
    protocol::step_stats(out, {0, 256, 1});
    protocol::cost_stats(out, CostStats{9, 8, 7, 6, 5, 4, 3, 2});
    RunnerStats s;
    s.live_sequences = 3;
    s.prefix_evictions = 25;
    protocol::stats(out, s);
    protocol::error(out, "x y");
    EXPECT(out.str() ==
           "READY MINIPREFIX 3 49152 0 2048 hip\nOK\nOK 0\nOK 1 -2.50000003e-08 3.14159274 65504 inf\n"
           "OK 2 r1 7 1 r2 -1 2\nOK 0 256 1\nOK 9 8 7 6 5 4 3 2\n"
           "OK 3 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0 25\nERROR x y\n");
}

// Records what the session asks of the runner; append returns logits with
// their maximum at (position of the sequence) % vocabulary.
class Recorder final : public ModelRunner {
public:
    ModelConfig cfg;
    std::map<RequestId, int> length, created;
    bool broken = false;
    int flushed = 0;
    Recorder() {
        cfg.context = 32;
        cfg.vocabulary = 4;
    }
    const ModelConfig& config() const override { return cfg; }
    int context_limit() const override { return cfg.context; }
    void create(const RequestId& id) override {
        if (length.count(id)) throw std::runtime_error("duplicate sequence");
        length[id] = 0;
        ++created[id];
    }
    std::vector<float> append(const RequestId& id, const std::vector<TokenId>& tokens) override {
        if (broken) throw std::runtime_error("device lost");
        auto it = length.find(id);
        if (it == length.end()) throw std::runtime_error("unknown sequence");
        for (TokenId t : tokens)
            if (t < 0 || t >= cfg.vocabulary) throw std::runtime_error("invalid token");
        it->second += (int)tokens.size();
        std::vector<float> logits(cfg.vocabulary, 0.5F);
        logits[it->second % cfg.vocabulary] = 2.0F;
        return logits;
    }
    std::size_t reuse_prefix(const RequestId& id, const std::vector<TokenId>&) override {
        if (length.at(id)) throw std::runtime_error("nonempty sequence");
        return 0;
    }
    void release(const RequestId& id) override {
        if (!length.erase(id)) throw std::runtime_error("unknown sequence");
    }
    void clear() override { length.clear(); }
    void clear_prefix_cache() override { ++flushed; }
    RunnerStats stats() const override {
        RunnerStats s;
        s.live_sequences = length.size();
        return s;
    }
};

struct CountingBuffer : std::stringbuf {
    int syncs = 0;
    int sync() override {
        ++syncs;
        return 0;
    }
};

void session_transcript() {
    auto owned = std::make_unique<Recorder>();
    Recorder* runner = owned.get();
    Engine engine(std::move(owned), {2, 8, 4, 32});
    std::istringstream in(
        "SUBMIT 1 2 -1 3 0 1 2\n"
        "SUBMIT 2 1 3 1 1\n"
        "STEP\n"
        "STEP_STATS\n"
        "STEP\n"
        "FORWARD 5 2 1 1\n"
        "FORWARD 5 1 9\n"
        "REUSE 5 1 1\n"
        "RELEASE 5\n"
        "CLEAR_PREFIX\n"
        "STATS\n"
        "QUIT\n"
        "STEP\n");
    CountingBuffer buffer;
    std::ostream out(&buffer);
    EXPECT(protocol::serve(engine, in, out) == 0);
    // Request 1 (3 prompt tokens) gets token 3 % 4 = 3, then 4 % 4 = 0, and
    // ends at its limit of 2; request 2's one prompt token gives token 1 (not
    // its EOS 3) and it ends at its limit of 1. Diagnostic sequence 5 is
    // created once; its failed append keeps it.
    const std::string want =
        "OK\nOK\n"
        "OK 2 1 3 -1 2 1 1\n"
        "OK 0 4 0\n"
        "OK 1 1 0 1\n"
        "OK 0.5 0.5 2 0.5\n"
        "ERROR invalid token\n"
        "ERROR nonempty sequence\n"
        "OK\nOK\nOK 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0\nOK\n";
    if (buffer.str() != want) std::fprintf(stderr, "transcript:\n%s", buffer.str().c_str());
    EXPECT(buffer.str() == want);
    EXPECT(buffer.syncs == 12);  // one flush per command up to and including QUIT
    std::string rest;
    std::getline(in, rest);
    EXPECT(rest == "STEP");
    EXPECT(runner->created["reference/5"] == 1 && runner->flushed == 1);
}

void end_of_input_is_not_quit() {
    auto owned = std::make_unique<Recorder>();
    Recorder* runner = owned.get();
    Engine engine(std::move(owned), {1, 4, 4, 32});
    std::istringstream in("SUBMIT 1 3 -1 1 1\nSTEP");
    std::ostringstream out;
    EXPECT(protocol::serve(engine, in, out) == 0);
    EXPECT(out.str() == "OK\nOK 1 1 1 -1\n");
    EXPECT(runner->length.count("1") == 1);  // still live: the engine's destructor cleans up
}

void failed_engine_refuses_runner_commands() {
    auto owned = std::make_unique<Recorder>();
    Recorder* runner = owned.get();
    runner->broken = true;
    Engine engine(std::move(owned), {1, 4, 4, 32});
    std::istringstream in("SUBMIT 1 1 -1 1 1\nSTEP\nFORWARD 1 1 1\nREUSE 1 1 1\nCACHE 1\nRELEASE 1\nCLEAR_PREFIX\n"
                          "COST_TIMING 1\nSTATS\nSTEP_STATS\nCOST_STATS\n");
    std::ostringstream out;
    protocol::serve(engine, in, out);
    std::string want = "OK\nOK 1 1 -1 3\n";
    for (int i = 0; i < 6; ++i) want += "ERROR engine failed; create a new engine\n";
    want += "OK 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0 0\nOK 0 0 0\nOK 0 0 0 0 0 0 0 0\n";
    if (out.str() != want) std::fprintf(stderr, "failed engine:\n%s", out.str().c_str());
    EXPECT(out.str() == want);
    EXPECT(engine.failed() && runner->flushed == 0);
}

}  // namespace

int main() {
    parse_errors_in_validation_order();
    parse_accepts();
    response_lines();
    session_transcript();
    end_of_input_is_not_quit();
    failed_engine_refuses_runner_commands();
    if (failures) {
        std::fprintf(stderr, "%d failures\n", failures);
        return 1;
    }
    std::cout << "worker protocol tests passed\n";
    return 0;
}
