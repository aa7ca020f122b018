// f16 tiles, B given as [K, N], K a multiple of 64 (whole-step loads).
#include "tile_inst.h"

CMPEXT3_TILE_TU(launch_tile_f16_kn_whole, _Float16, true, false)
