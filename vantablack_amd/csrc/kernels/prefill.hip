// Causal prefill attention on MFMA (gfx950): placeholder module.
#include "common.h"
