// pmkl/pmkl.h - umbrella header of the MI355X attention path (reference
// pmkl/pmkl.h:1-6 includes core, the add/sub ops and causal attention; only
// the attention path and the core pieces it uses exist here).
#pragma once

#include "core.h"
#include "nlp/causal_attention.h"
