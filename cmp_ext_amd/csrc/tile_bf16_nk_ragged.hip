// bf16 tiles, B given as [N, K], K not a multiple of 64 (checked loads).
#include "tile_inst.h"

CMPEXT3_TILE_TU(launch_tile_bf16_nk_ragged, __bf16, false, true)
