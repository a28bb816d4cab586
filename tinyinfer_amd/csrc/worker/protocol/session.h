// Protocol v3 line loop (interface of miniprefix/apps/protocol/session.h):
// reads commands until QUIT or end of input, answers each with one line
// and a flush. Start-up (model load, READY) is the executable's part.
#pragma once
#include "miniprefix/engine.h"

#include <istream>
#include <ostream>

namespace miniprefix::protocol {

int serve(Engine&, std::istream&, std::ostream&);

}  // namespace miniprefix::protocol
