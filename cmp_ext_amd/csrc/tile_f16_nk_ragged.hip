// f16 tiles, B given as [N, K], K not a multiple of 64 (checked loads).
#include "tile_inst.h"

CMPEXT3_TILE_TU(launch_tile_f16_nk_ragged, _Float16, false, true)
