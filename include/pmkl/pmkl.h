// pmkl/pmkl.h - umbrella header of the MI355X attention path (reference
// pmkl/pmkl.h:1-6 includes core, the add/sub ops and causal attention; here:
// the attention path, the row softmax and the core pieces they use).
#pragma once

#include "core.h"
#include "dtype.h"
#include "nlp/causal_attention.h"
#include "norm/warp_softmax.h"
