// Protocol v3 of the MiniPrefix worker: command parsing, the response lines
// and the session loop with its diagnostic sequences. The wire format is the
// reference worker's (miniprefix/apps/protocol/command.cpp, response.cpp,
// session.cpp, diagnostics.cpp); existing clients
// (miniprefix/bindings/python/client.py) drive this worker unchanged.
#include "protocol/command.h"
#include "protocol/response.h"
#include "protocol/session.h"

#include <cstdio>
#include <functional>
#include <map>
#include <set>
#include <sstream>
#include <stdexcept>

namespace miniprefix::protocol {
namespace {

constexpr int kMaxTokens = 131072;

// The fields of one command line, consumed left to right.
class Fields {
public:
    explicit Fields(const std::string& line) : in_(line) {}
    std::string word() {
        std::string w;
        in_ >> w;
        return w;
    }
    int number() {
        int v = 0;
        if (!(in_ >> v)) throw std::invalid_argument("missing integer");
        return v;
    }
    std::vector<TokenId> tokens(int count) {
        if (count < 1 || count > kMaxTokens) throw std::invalid_argument("invalid token count");
        std::vector<TokenId> out;
        out.reserve(count);
        while ((int)out.size() < count) out.push_back(number());
        return out;
    }

private:
    std::istringstream in_;
};

Command submit_command(Fields& f) {
    // All four header fields are read before any of them is judged.
    const int id = f.number(), limit = f.number(), eos = f.number(), count = f.number();
    if (id < 1 || limit < 1) throw std::invalid_argument("invalid request");
    Command c{Kind::Submit};
    c.request.id = std::to_string(id);
    c.request.prompt_token_ids = f.tokens(count);
    c.request.generation.max_new_tokens = limit;
    if (eos >= 0)
        c.request.generation.eos_token_id = eos;
    else if (eos != -1)
        throw std::invalid_argument("invalid EOS");
    return c;
}

Command sequence_command(Fields& f, Kind kind) {
    Command c{kind};
    c.id = f.number();
    const int count = f.number();
    c.input = f.tokens(count);
    if (c.id < 1) throw std::invalid_argument("invalid diagnostic sequence");
    return c;
}

Command id_command(Fields& f, Kind kind) {
    Command c{kind};
    c.id = f.number();
    return c;
}

Command timing_command(Fields& f) {
    Command c{Kind::CostTiming};
    c.id = f.number();
    if (c.id != 0 && c.id != 1) throw std::invalid_argument("invalid timing flag");
    return c;
}

using Parser = std::function<Command(Fields&)>;

const std::map<std::string, Parser>& parsers() {
    static const std::map<std::string, Parser> table = {
        {"SUBMIT", submit_command},
        {"FORWARD", [](Fields& f) { return sequence_command(f, Kind::Forward); }},
        {"REUSE", [](Fields& f) { return sequence_command(f, Kind::Reuse); }},
        {"CANCEL", [](Fields& f) { return id_command(f, Kind::Cancel); }},
        {"CACHE", [](Fields& f) { return id_command(f, Kind::Cache); }},
        {"RELEASE", [](Fields& f) { return id_command(f, Kind::Release); }},
        {"COST_TIMING", timing_command},
        {"STEP", [](Fields&) { return Command{Kind::Step}; }},
        {"STEP_STATS", [](Fields&) { return Command{Kind::StepStats}; }},
        {"CLEAR_PREFIX", [](Fields&) { return Command{Kind::ClearPrefix}; }},
        {"COST_STATS", [](Fields&) { return Command{Kind::CostStats}; }},
        {"STATS", [](Fields&) { return Command{Kind::Stats}; }},
        {"QUIT", [](Fields&) { return Command{Kind::Quit}; }},
    };
    return table;
}

// Diagnostic sequences live in their own id space ("reference/<id>") beside
// the engine's requests and are created on first use. A failed append or
// reuse keeps a sequence that was created; a release forgets it only once
// the runner has released it.
class Diagnostics {
public:
    explicit Diagnostics(ModelRunner& runner) : runner_(runner) {}
    std::vector<float> forward(int id, const std::vector<TokenId>& tokens) {
        return runner_.append(open(id), tokens);
    }
    std::size_t reuse(int id, const std::vector<TokenId>& tokens) { return runner_.reuse_prefix(open(id), tokens); }
    void cache(int id) { runner_.cache_prefix(name(id)); }
    void release(int id) {
        const std::string n = name(id);
        runner_.release(n);
        open_.erase(n);
    }
    void clear_prefix() { runner_.clear_prefix_cache(); }

private:
    static std::string name(int id) { return "reference/" + std::to_string(id); }
    std::string open(int id) {
        std::string n = name(id);
        if (!open_.count(n)) {
            runner_.create(n);
            open_.insert(n);
        }
        return n;
    }
    ModelRunner& runner_;
    std::set<std::string> open_;
};

// Commands that use the runner directly must not touch a backend whose
// engine has failed.
bool needs_healthy_runner(Kind k) {
    return k == Kind::Forward || k == Kind::Reuse || k == Kind::Cache || k == Kind::Release ||
           k == Kind::ClearPrefix || k == Kind::CostTiming;
}

// Runs one command and writes its response; true after QUIT.
bool run(Engine& engine, Diagnostics& diagnostics, Command& c, std::ostream& out) {
    if (engine.failed() && needs_healthy_runner(c.kind)) throw std::runtime_error("engine failed; create a new engine");
    switch (c.kind) {
    case Kind::Submit: engine.submit(std::move(c.request)); ok(out); break;
    case Kind::Step: engine.step(); events(out, engine.poll_events()); break;
    case Kind::StepStats: step_stats(out, engine.last_step_stats()); break;
    case Kind::Cancel: engine.cancel(std::to_string(c.id)); events(out, engine.poll_events()); break;
    case Kind::ClearPrefix: diagnostics.clear_prefix(); ok(out); break;
    case Kind::Cache: diagnostics.cache(c.id); ok(out); break;
    case Kind::Reuse: count(out, diagnostics.reuse(c.id, c.input)); break;
    case Kind::Forward: logits(out, diagnostics.forward(c.id, c.input)); break;
    case Kind::Release: diagnostics.release(c.id); ok(out); break;
    case Kind::CostStats: cost_stats(out, engine.runner().cost_stats()); break;
    case Kind::CostTiming: engine.runner().set_cost_timing(c.id != 0); ok(out); break;
    case Kind::Stats: stats(out, engine.runner().stats()); break;
    case Kind::Quit: engine.shutdown(); ok(out); return true;
    }
    return false;
}

template <typename... T>
void fields(std::ostream& out, const T&... values) {
    out << "OK";
    ((out << ' ' << values), ...);
    out << '\n';
}

}  // namespace

Command parse(const std::string& line) {
    Fields f(line);
    const auto& table = parsers();
    const auto it = table.find(f.word());
    if (it == table.end()) throw std::invalid_argument("unknown command");
    return it->second(f);
}

void ready(std::ostream& out, int vocabulary, int eos, int context, const std::string& backend) {
    out << "READY MINIPREFIX 3 " << vocabulary << ' ' << eos << ' ' << context << ' ' << backend << '\n' << std::flush;
}

void ok(std::ostream& out) { out << "OK\n"; }

void count(std::ostream& out, std::size_t value) { fields(out, value); }

void logits(std::ostream& out, const std::vector<float>& values) {
    // Nine significant digits, shortest form (the stream's default float
    // format at precision 9): every float round-trips.
    out << "OK";
    char text[32];
    for (float v : values) {
        std::snprintf(text, sizeof text, " %.9g", (double)v);
        out << text;
    }
    out << '\n';
}

void events(std::ostream& out, const std::vector<GenerationEvent>& batch) {
    out << "OK " << batch.size();
    for (const GenerationEvent& e : batch)
        out << ' ' << e.request_id << ' ' << (e.token_id ? *e.token_id : -1) << ' '
            << (e.finish_reason ? static_cast<int>(*e.finish_reason) : -1);
    out << '\n';
}

void cost_stats(std::ostream& out, const CostStats& s) {
    fields(out, s.lookup_calls, s.lookup_ns, s.publish_calls, s.publish_ns, s.cow_pages, s.cow_bytes, s.cow_copy_ns,
           s.cow_timed_copies);
}

void stats(std::ostream& out, const RunnerStats& s) {
    fields(out, s.live_sequences, s.live_kv_bytes, s.peak_kv_bytes, s.forward_tokens, s.device_weight_bytes,
           s.weight_uploaded_bytes, s.token_uploaded_bytes, s.kv_uploaded_bytes, s.logits_downloaded_bytes,
           s.device_allocations, s.device_workspace_bytes, s.kv_block_tokens, s.kv_total_blocks, s.kv_live_blocks,
           s.kv_peak_blocks, s.kv_reserved_bytes, s.block_table_uploaded_bytes, s.block_table_device_bytes,
           s.prefix_cache_capacity, s.kv_cached_blocks, s.kv_cache_only_blocks, s.prefix_hits, s.prefix_misses,
           s.prefix_reused_tokens, s.prefix_evictions);
}

void step_stats(std::ostream& out, const EngineStepStats& s) {
    fields(out, s.prefix_reused_tokens, s.prefill_tokens, s.decode_tokens);
}

void error(std::ostream& out, const std::string& message) { out << "ERROR " << message << '\n'; }

int serve(Engine& engine, std::istream& in, std::ostream& out) {
    Diagnostics diagnostics(engine.runner());
    std::string line;
    while (std::getline(in, line)) {
        bool quit = false;
        try {
            Command c = parse(line);
            quit = run(engine, diagnostics, c, out);
        } catch (const std::exception& e) {
            error(out, e.what());
        }
        out << std::flush;
        if (quit) return 0;
    }
    return 0;
}

}  // namespace miniprefix::protocol
