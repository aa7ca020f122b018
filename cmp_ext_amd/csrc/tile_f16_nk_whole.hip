// f16 tiles, B given as [N, K], K a multiple of 64 (whole-step loads).
#include "tile_inst.h"

CMPEXT3_TILE_TU(launch_tile_f16_nk_whole, _Float16, false, false)
