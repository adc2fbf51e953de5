// Instantiates every forward and backward kernel of one hidden size, so that
// the build compiles the six hidden sizes as separate translation units in
// parallel. Compiled once per size with -DRLN_HIDDEN=<H>.
#include "rln_device.h"

#ifndef RLN_HIDDEN
#error "compile with -DRLN_HIDDEN=<hidden size>"
#endif

namespace rln {

template int launch_forward_hidden<RLN_HIDDEN>(const ForwardArgs&, int, int, bool);
template int launch_backward_hidden<RLN_HIDDEN>(const BackwardArgs&, int, int, bool);

}  // namespace rln
