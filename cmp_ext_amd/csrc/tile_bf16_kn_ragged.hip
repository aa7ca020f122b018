// bf16 tiles, B given as [K, N], K not a multiple of 64 (checked loads).
#include "tile_inst.h"

CMPEXT3_TILE_TU(launch_tile_bf16_kn_ragged, __bf16, true, true)
