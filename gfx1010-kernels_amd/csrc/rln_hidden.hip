// Instantiates the forward and backward kernels of one row shape, so that
// the build compiles the shapes as separate translation units in parallel.
// Compiled once per shape, with -DRLN_HIDDEN=<H> for a specialized hidden
// size or -DRLN_WIDE_V=<V> -DRLN_WIDE_P=<P> for a run-time one, and
// -DRLN_PASSES=<1: forward, 2: backward, 3: both> for the passes that run
// the shape (both when not given).
#include "rln_device.h"

#if defined(RLN_HIDDEN)
#define RLN_SHAPE FixedShape<RLN_HIDDEN>
#elif defined(RLN_WIDE_V) && defined(RLN_WIDE_P)
#define RLN_SHAPE WideShape<RLN_WIDE_V, RLN_WIDE_P>
#else
#error "compile with -DRLN_HIDDEN=<H> or -DRLN_WIDE_V=<V> -DRLN_WIDE_P=<P>"
#endif
#if !defined(RLN_PASSES)
#define RLN_PASSES 3
#endif

namespace rln {

#if RLN_PASSES & 1
template int launch_forward_shape<RLN_SHAPE>(const ForwardArgs&, RLN_SHAPE, int, int, bool);
#endif
#if RLN_PASSES & 2
template int launch_backward_shape<RLN_SHAPE>(const BackwardArgs&, RLN_SHAPE, int, int, bool);
#if defined(RLN_HIDDEN) && RLN_HIDDEN == 768
template int launch_backward_shape<TwelveWaveShape<768>>(const BackwardArgs&,
                                                         TwelveWaveShape<768>, int, int, bool);
#endif
#if defined(RLN_HIDDEN) && RLN_HIDDEN == 384
template int launch_backward_shape<NineWaveShape<384>>(const BackwardArgs&,
                                                       NineWaveShape<384>, int, int, bool);
#endif
#if defined(RLN_WIDE_P) && RLN_WIDE_P == 4 && RLN_WIDE_V <= 2
template int launch_backward_shape<StaggeredWideShape<RLN_WIDE_V>>(
    const BackwardArgs&, StaggeredWideShape<RLN_WIDE_V>, int, int, bool);
#endif
#endif

}  // namespace rln
