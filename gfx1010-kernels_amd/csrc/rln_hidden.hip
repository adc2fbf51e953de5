// Instantiates every forward and backward kernel of one row shape, so that
// the build compiles the shapes as separate translation units in parallel.
// Compiled once per shape, with -DRLN_HIDDEN=<H> for a specialized hidden
// size or -DRLN_WIDE_V=<V> -DRLN_WIDE_P=<P> for a run-time one.
#include "rln_device.h"

#if defined(RLN_HIDDEN)
#define RLN_FORWARD_SHAPE FixedShape<RLN_HIDDEN>
#define RLN_BACKWARD_SHAPE FixedShape<RLN_HIDDEN>
#elif defined(RLN_WIDE_V) && defined(RLN_WIDE_P)
#define RLN_FORWARD_SHAPE WideShape<RLN_WIDE_V, RLN_WIDE_P>
#define RLN_BACKWARD_SHAPE WideShape<RLN_WIDE_V, RLN_WIDE_P>
#else
#error "compile with -DRLN_HIDDEN=<H> or -DRLN_WIDE_V=<V> -DRLN_WIDE_P=<P>"
#endif

namespace rln {

template int launch_forward_shape<RLN_FORWARD_SHAPE>(const ForwardArgs&, RLN_FORWARD_SHAPE, int,
                                                     int, bool);
template int launch_backward_shape<RLN_BACKWARD_SHAPE>(const BackwardArgs&, RLN_BACKWARD_SHAPE,
                                                       int, int, bool);

}  // namespace rln
