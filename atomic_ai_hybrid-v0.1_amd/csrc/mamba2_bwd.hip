// Mamba2 SSD chunk-scan backward for gfx950.
#include "mamba2_fwd.hip"
