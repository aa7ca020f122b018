// Host-side kernel selector: argument validation, kernel choice and launch
// geometry for every GEMM request.  The reference fixes one tile per dtype
// at compile time (src/cuda/fp16_matmul.cu:12-22, bf16_matmul.cu:11-21,
// fp32_matmul.cu:10-14); here the choice depends on dtype, M/N/K, layout and
// alignment.
#include "selector.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>

#include "../../include/cmpext3_gemm.h"

namespace cmpext3 {
namespace {

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

struct Candidate {
  KernelId id;
  int bm, bn;
  int occ;      // workgroups a CU runs at once (1 unless the kernel is built for more)
  double eff;   // relative per-flop throughput of a CU running occ of these tiles (measured)
  double eff1;  // the same with one workgroup on the CU (latency-bound; = eff when occ == 1)
};

// Modelled cost of a tiled product, optionally with K split s ways (fp32 partials
// summed, biased and rounded by a second launch): tiles go out in rounds of
// kNumCUs * occ (workgroups are handed out as slots free, and a CU's matrix cores
// are shared by whatever it holds); a round is worth occ * bm * bn * (K per split) /
// eff on the busiest CU (measured on MI355X, this tracks the fp32 and 16-bit tile
// kernels across 512^3 .. 4096^3 and ragged shapes), except that a last round leaving
// every CU a single workgroup is worth bm * bn * (K per split) / eff1; a split adds
// writing and reading the partials at ~5 TB/s and ~6 us for the extra launch.  Units
// per microsecond on MI355X: one round of 256x256 16-bit tiles at K = 4096 takes ~102 us.
constexpr double kUnitsPerUs = 65536.0 * 4096.0 / 102.0;
double split_cost(const Candidate& c, int64_t M, int64_t N, int64_t K, int64_t batch, int64_t s,
                  double units_per_us = kUnitsPerUs) {
  const int64_t tiles = cdiv(M, c.bm) * cdiv(N, c.bn) * batch;
  const int64_t slots = (int64_t)kNumCUs * c.occ, wgs = tiles * s;
  const int64_t full = wgs / slots, rem = wgs - full * slots;
  const double tile = (double)c.bm * c.bn * (double)cdiv(K, s);
  double gemm = (double)full * c.occ * tile / c.eff;
  if (rem > 0) gemm += rem <= kNumCUs ? tile / c.eff1 : c.occ * tile / c.eff;
  const double reduce = s > 1 ? ((double)s * batch * M * N * 8.0 / 5e6 + 6.0) * units_per_us : 0.0;
  return gemm + reduce;
}


// Per-area throughput of a CU running the tile, relative to 256x256 (MI355X, fp16
// 4096^3: 256x256 102.7 us, 128x128 with two workgroups per CU 126.7 us; one 128x128
// workgroup alone on its CU: 128 x 4096 x 4096 unsplit 41.5 us, 8 x 2048 x 128 x 2048
// 24.1 us, i.e. 0.61 and 0.53).
const Candidate kTiles16[] = {
    {kTile256x256, 256, 256, 1, 1.00, 1.00},
    {kTile256x224, 256, 224, 1, 0.98, 0.98},
    {kTile128x128, 128, 128, 2, 0.81, 0.57},
};
// fp32 tiles.  A CU holds up to `occ` of their workgroups at once and shares its
// matrix cores among them; how busy it keeps them grows with the number it holds:
// from u1 (one workgroup, latency-bound) to umax (occ of them).  Fitted on MI355X to
// 345 timed (tile, K split) choices over 27 shapes (M 16..4097, N 1024..4096, K
// 1024..14336): the model's choice is within 1.7 % of the fastest measured one
// (geometric mean; worst 1.18x at 1024^3), against 1.12x for a model with a fixed
// per-tile efficiency.  The 4-byte LDS-DMA path (rows not 16-byte aligned) scales
// umax by dma4, measured per tile at full occupancy against the 16-byte path on the
// same box: 128x128 505 vs 539 us, 96x64 412 vs 423, 64x64 270 vs 321.  64x64k4 (K
// split over the four waves, two workgroups per CU) fitted the same way to 114 more
// timings: u1 0.62, umax 0.72; with it the model's choice is within 0.4 % of the
// fastest measured (tile, split) over those 29 shapes.  16x64k4 (M <= 16, bound by
// streaming B) to 134 more over 29 shapes with M <= 16: u1 0.36, umax 0.46, and a CU
// streams its workgroups' B strips at ~19 GB/s with one of them, ~24 GB/s with more
// (6 TB/s over 256 CUs); the choice is then within 2.7 % of the fastest measured.
struct F32Tile {
  KernelId id;
  int bm, bn, occ;
  double u1, umax, dma4;
  int kwaves;  // waves that split a workgroup's 16-k steps among them
};
const F32Tile kTiles32[] = {
    {kF32Tile128, 128, 128, 4, 0.75, 0.94, 0.937, 1},
    {kF32Tile96x64, 96, 64, 8, 0.50, 0.89, 0.975, 1},
    {kF32Tile64, 64, 64, 8, 0.44, 0.875, 0.84, 1},
    {kF32Tile64K4, 64, 64, 2, 0.62, 0.72, 0.84, 4},
    {kF32Tile16K4, 16, 64, 4, 0.36, 0.46, 0.84, 4},
};
// Modelled microseconds: w = workgroups on the busiest CU, each running cdiv(K/s, 16)
// steps of bm*bn*16 MFMA work (bm*bn*32 / (256 * 2380) us at the full fp32 rate of a
// CU at 2.38 GHz), but no less than streaming A and B once at ~5.4 TB/s, nor than the
// busiest CU streaming its workgroups' B strips (bn columns over their K range); a split
// adds its fp32 partials written and read back at ~5.5 TB/s plus ~3.8 us.
double f32_cost(const F32Tile& c, int64_t M, int64_t N, int64_t K, int64_t batch, int64_t s, bool dma16) {
  const int64_t w = cdiv(cdiv(M, c.bm) * cdiv(N, c.bn) * batch * s, (int64_t)kNumCUs);
  const double steps = (double)(cdiv(cdiv(cdiv(K, s), 16), c.kwaves) * c.kwaves);
  const double step_us = c.bm * c.bn * 32.0 / (256.0 * 2380.0);
  const double umax = dma16 ? c.umax : c.dma4 * c.umax;
  const double u = c.u1 + (umax - c.u1) * std::min(1.0, (double)(w - 1) / (c.occ - 1));
  const double mem = std::max((double)batch * (M * K + K * N) * 4.0 / 5.4e6,
                              (double)w * c.bn * cdiv(K, s) * 4.0 / (w == 1 ? 19e3 : 24e3));
  double t = 1.0 + std::max((double)w * steps * step_us / u, mem);
  if (s > 1) t += (double)s * batch * M * N * 8.0 / 5.5e6 + 3.8;
  return t;
}

const char* kernel_name(KernelId id) {
  switch (id) {
    case kTile256x256: return "tile256x256";
    case kTile256x224: return "tile256x224";
    case kTile128x128: return "tile128x128";
    case kTile64x256: return "tile64x256";
    case kSkinny: return "skinny";
    case kSkinnyWide: return "skinny_wide";
    case kSkinnyNK: return "skinny_nk";
    case kF32Tile128: return "f32tile128x128";
    case kF32Tile64: return "f32tile64x64";
    case kF32Tile96x64: return "f32tile96x64";
    case kF32Tile64K4: return "f32tile64x64k4";
    case kF32Tile16K4: return "f32tile16x64k4";
    case kGeneric16: return "generic64x64";
    case kStream64x128: return "stream64x128";
    case kTall: return "tall";
    case kStream128x128: return "stream128x128";
    default: return "?";
  }
}

}  // namespace

namespace {
// Tuning override: CMPEXT3_GEMM_CONFIG="kernel=<name>[,splits=<s>][,strip=<rows>]" (names as in the plan
// strings, e.g. tile128x128, stream64x128, generic64x64, f32tile96x64) replaces the
// selector's choice wherever that kernel's own requirements hold for the call; otherwise,
// and for an unknown name or malformed value, it is ignored.  Read on every plan, so a
// tuning sweep can change it between calls.  For sweeps only: the selector's choices are
// the measured ones.
struct Override {
  int kernel = -1;
  int splits = 1;
  int strip = 0;  // rows of A (tall: 32 or 64) or of W (skinny_nk: 16, 32 or 64) per workgroup; 0: the selector's
};

Override read_override() {
  Override o;
  const char* env = getenv("CMPEXT3_GEMM_CONFIG");
  if (env == nullptr) return o;
  char buf[128];
  snprintf(buf, sizeof buf, "%s", env);
  char* save = nullptr;  // strtok_r: plans may be made on several host threads at once
  for (char* tok = strtok_r(buf, ", ", &save); tok != nullptr; tok = strtok_r(nullptr, ", ", &save)) {
    if (strncmp(tok, "kernel=", 7) == 0) {
      for (int id = 0; id < kNumKernels; ++id)
        if (strcmp(tok + 7, kernel_name((KernelId)id)) == 0) o.kernel = id;
    } else if (strncmp(tok, "splits=", 7) == 0) {
      const int v = atoi(tok + 7);
      if (v >= 1 && v <= 16) o.splits = v;
    } else if (strncmp(tok, "strip=", 6) == 0) {
      const int v = atoi(tok + 6);
      if (v == 16 || v == 32 || v == 64) o.strip = v;
    }
  }
  return o;
}

// K split of a forced tile kernel: s ways (ranges of whole 64-k steps, none empty), fp32
// partials in the workspace (N % 4 == 0 for their 16-byte stores); 1 if that does not fit.
int forced_splits(const Request& r, int s, int64_t* ksplit) {
  if (s <= 1 || r.N % 4 != 0 || r.K <= 0) return 1;
  const int64_t ks = cdiv(cdiv(r.K, s), 64) * 64;
  if ((s - 1) * ks >= r.K || (int64_t)s * r.batch * r.M * r.N * 4 > r.ws_bytes) return 1;
  *ksplit = ks;
  return s;
}

// K split of a strips kernel (skinny_nk, tall): ranges of whole 256-k stages, none empty,
// fp32 partials [split][batch][M][N] in the workspace (their 16-byte stores need N % 4 ==
// 0); left unsplit when the workspace is too small.
void split_strips(const Request& r, int64_t splits, Plan* q) {
  if (splits <= 1 || r.N % 4 != 0 || r.K <= 256) return;
  const int64_t ks = cdiv(cdiv(r.K, splits), 256) * 256;
  const int64_t s = cdiv(r.K, ks);
  const int64_t need = s * r.batch * r.M * r.N * 4;
  if (s > 1 && need <= r.ws_bytes) {
    q->splits = (int)s;
    q->ksplit = (int)ks;
    q->ws_bytes = need;
  }
}

// skinny_nk (M <= 64, B as [N, K]): strips of W rows over all of K, or over K ranges of
// `splits` (fp32 partials in the workspace, N % 4 == 0; a split that does not fit the
// workspace is dropped).  16-row strips when 32-row ones would leave CUs idle.  With more
// than 16 rows of A every workgroup re-reads all of A from L2 (for 64 x 4096: twice W's
// bytes over 448 strips of a 14336-row W), so 64-row strips there once they still give
// >= 192 workgroups (MI355X, x[M, 4096] W[14336, 4096]^T: M = 32 27.7 -> 23.9 us, 48 30.2
// -> 26.8, 64 34.1 -> 29.3; x[64, 8192] W[14336, 8192]^T 56.8 -> 51.6; x[64, 8192]
// W[28672, 8192]^T 111 either way).
Plan skinny_nk_plan(const Request& r, int64_t splits, int group_m) {
  Plan q{};
  q.kernel = kSkinnyNK;
  q.group_m = group_m;
  q.threads = 256;
  q.splits = 1;
  q.mb = (int)std::max<int64_t>(1, cdiv(r.M, 16));
  q.bm = 16 * q.mb;
  const int64_t chunk = std::min<int64_t>(r.batch, 65535);
  q.bn = cdiv(r.N, 32) * chunk >= kNumCUs ? 32 : 16;
  if (q.mb >= 2 && cdiv(r.N, 64) * chunk >= 192) q.bn = 64;
  split_strips(r, splits, &q);
  return q;
}

// The tall kernel for N <= 128 (16-row blocks of B's columns: 4 up to 64 columns, else 8;
// for B as [N, K] 1 up to 16 and 2 up to 32) with strips of `strip` rows of A, over all of
// K or over K ranges of `splits`.
Plan tall_plan(const Request& r, int strip, int group_m, int64_t splits = 1) {
  Plan q{};
  q.kernel = kTall;
  q.group_m = group_m;
  q.threads = 256;
  q.splits = 1;
  q.mb = r.N <= 64 ? 4 : 8;
  if (r.layout == kNK && r.N <= 32) q.mb = r.N <= 16 ? 1 : 2;  // B as [N, K]: 16-row blocks as needed
  q.bm = strip;
  q.bn = 16 * q.mb;
  split_strips(r, splits, &q);
  return q;
}

// Applies the override to a 16-bit plan: a tiled kernel (optionally split) when `fast`,
// the streaming kernel when `stream_ok`, the tall kernel when `tall_ok`, skinny_nk
// (optionally split) when `skinny_nk_ok`, the generic kernel always.
void override16(const Request& r, bool fast, bool stream_ok, bool tall_ok, bool skinny_nk_ok, Plan* p) {
  const Override o = read_override();
  if (o.kernel < 0) return;
  Plan q{};
  q.group_m = p->group_m;
  q.threads = 256;
  q.splits = 1;
  switch (o.kernel) {
    case kTile256x256:
    case kTile256x224:
    case kTile128x128:
    case kTile64x256: {
      if (!fast) return;
      q.kernel = (KernelId)o.kernel;
      q.bm = o.kernel == kTile64x256 ? 64 : o.kernel == kTile128x128 ? 128 : 256;
      q.bn = o.kernel == kTile256x224 ? 224 : o.kernel == kTile128x128 ? 128 : 256;
      if (q.bm == 256) q.threads = 512;
      int64_t ks = 0;
      if (q.bm >= 128 && (q.splits = forced_splits(r, o.splits, &ks)) > 1) {
        q.ksplit = (int)ks;
        q.ws_bytes = (int64_t)q.splits * r.batch * r.M * r.N * 4;
      }
      break;
    }
    case kStream64x128:
    case kStream128x128:
      if (!stream_ok) return;
      q.kernel = r.M <= 64 ? kStream64x128 : kStream128x128;
      q.bm = r.M <= 64 ? 64 : 128;
      q.bn = 128;
      q.threads = r.M <= 64 ? 256 : 512;
      break;
    case kGeneric16:
      q.kernel = kGeneric16;
      q.bm = 64;
      q.bn = 64;
      q.forced = true;  // no padded copies in its place
      break;
    case kSkinnyNK:
      if (!skinny_nk_ok) return;
      q = skinny_nk_plan(r, o.splits, p->group_m);
      if (o.strip) q.bn = o.strip;
      break;
    case kTall:
      // strips of 32 or 64 rows of A only (0: 64); a 16-row strip is not built for it
      if (!tall_ok || o.strip == 16) return;
      q = tall_plan(r, o.strip == 32 ? 32 : 64, p->group_m, o.splits);
      break;
    default:
      return;
  }
  *p = q;
}

// Applies the override to an fp32 plan: any fp32 tile, optionally split.
void override32(const Request& r, bool dma16, Plan* p) {
  const Override o = read_override();
  if (o.kernel < 0) return;
  for (const F32Tile& c : kTiles32) {
    if (c.id != o.kernel) continue;
    Plan q{};
    q.group_m = p->group_m;
    q.threads = 256;
    q.kernel = c.id;
    q.bm = c.bm;
    q.bn = c.bn;
    q.dma16 = dma16;
    int64_t ks = 0;
    if ((q.splits = forced_splits(r, o.splits, &ks)) > 1) {
      q.ksplit = (int)ks;
      q.ws_bytes = (int64_t)q.splits * r.batch * r.M * r.N * 4;
    }
    q.forced = true;  // no padded copies in its place
    *p = q;
  }
}

int make_plan_core(const Request& r, Plan* plan) {
  if (r.dtype != kF16 && r.dtype != kBF16 && r.dtype != kF32) return CMPEXT3_ERR_UNSUPPORTED;
  if (r.layout != kKN && r.layout != kNK) return CMPEXT3_ERR_UNSUPPORTED;
  if (r.M < 0 || r.N < 0 || r.K < 0 || r.batch < 0) return CMPEXT3_ERR_INVALID_ARG;
  const int64_t kIntMax = 0x7FFFFFFF;
  if (r.M > kIntMax || r.N > kIntMax || r.K > kIntMax) return CMPEXT3_ERR_TOO_LARGE;
  const int64_t b_cols = r.layout == kKN ? r.N : r.K;
  if (r.lda < std::max<int64_t>(1, r.K) || r.ldb < std::max<int64_t>(1, b_cols) ||
      r.ldc < std::max<int64_t>(1, r.N))
    return CMPEXT3_ERR_INVALID_ARG;
  if (r.batch > 1 && (r.stride_a < 0 || r.stride_b < 0 || r.stride_c < 0)) return CMPEXT3_ERR_INVALID_ARG;
  const int64_t esz = r.dtype == kF32 ? 4 : 2;
  // Kernels address at most 256 rows of an operand from a per-tile base with
  // 32-bit byte offsets.
  if (256 * r.lda * esz > kIntMax || 256 * r.ldb * esz > kIntMax) return CMPEXT3_ERR_TOO_LARGE;
  // The fp32 kernels store C the same way (the 16-bit ones through 64-bit pointers).
  if (r.dtype == kF32 && 256 * r.ldc * esz > kIntMax) return CMPEXT3_ERR_TOO_LARGE;
  if (cdiv(r.M, 64) * cdiv(r.N, 64) > kIntMax) return CMPEXT3_ERR_TOO_LARGE;

  Plan p{};
  p.group_m = 4;
  p.threads = 256;
  const bool batched = r.batch > 1;
  if (r.dtype == kF32) {
    // tile and K split with the lowest modelled cost, as for 16-bit products below (fp32
    // has no skinny kernel, so few-tile products of any M split K; >= 16 K steps each)
    const bool dma16 = (r.align_a ? r.align_a : r.align) >= 16 && (r.align_b ? r.align_b : r.align) >= 16 &&
                       r.K % 4 == 0 && r.lda % 4 == 0 && r.ldb % 4 == 0 &&
                       (r.layout == kNK || r.N % 4 == 0 || r.b_cols_padded) &&
                       (!batched || (r.stride_a % 4 == 0 && r.stride_b % 4 == 0));
    const F32Tile* best = &kTiles32[0];
    int64_t best_s = 1;
    double best_cost = -1.0;
    for (const F32Tile& c : kTiles32) {
      if (c.bm == 16 && r.M > 16) continue;  // 16-row tiles: measured and meant for M <= 16 only
      const int64_t smax = (r.N % 4 == 0 && r.K >= 1024) ? std::min<int64_t>(16, r.K / 256) : 1;
      for (int64_t s = 1; s <= std::max<int64_t>(1, smax); ++s) {
        if (s > 1 && s * r.batch * r.M * r.N * 4 > r.ws_bytes) break;
        const double cost = f32_cost(c, r.M, r.N, r.K, r.batch, s, dma16);
        if (best_cost < 0 || cost < best_cost) {
          best_cost = cost;
          best = &c;
          best_s = s;
        }
      }
    }
    p.kernel = best->id;
    p.bm = best->bm;
    p.bn = best->bn;
    p.dma16 = dma16;
    if (best_s > 1) {
      p.splits = (int)best_s;
      p.ksplit = (int)(cdiv(cdiv(r.K, best_s), 64) * 64);
      p.ws_bytes = best_s * r.batch * r.M * r.N * 4;
    }
    override32(r, dma16, &p);
  } else {
    const bool skinny_ok = r.M <= 64 && r.align >= 16 && r.K % 8 == 0 &&
                           r.lda % 8 == 0 && r.N % 8 == 0 && r.ldb % 8 == 0 &&
                           (!batched || (r.stride_a % 8 == 0 && r.stride_b % 8 == 0));
    // (the tiled kernels' epilogue stores in 16-, 8- or 2-byte pieces as C's rows allow)
    const bool fast = r.align >= 16 && r.K % 8 == 0 && r.lda % 8 == 0 && r.ldb % 8 == 0 &&
                      (r.layout == kNK || r.N % 8 == 0 || r.b_cols_padded) &&
                      (!batched || (r.stride_a % 8 == 0 && r.stride_b % 8 == 0));
    // With M <= 64 the skinny kernels pay off only where the GPU would otherwise
    // starve: once 128-column tiles alone give every CU one (N >= 32768, or a
    // batch of such products, e.g. a 1x1 convolution over many pixels), the tiled
    // kernel streams B faster (MI355X, 128x128 tile vs unsplit skinny kernel:
    // 64x1048576x128 118 vs 237 us, 16x262144x512 48 vs 67 us, 64x32768x128 5.5
    // vs 8.3 us).
    const bool skinny_tiles_enough = fast && cdiv(r.N, 128) * r.batch >= kNumCUs;
    // what the streaming kernel needs (one A for the batch, C's rows in 16-byte pieces, ...;
    // B as [K,N] or [N,K]; it is chosen below only with enough tiles per workgroup)
    const bool stream_ok = fast && r.M <= kStreamMaxRows && r.K <= 256 && r.N % 8 == 0 &&
                           r.ldc % 8 == 0 && (!batched || (r.stride_a == 0 && r.stride_c % 8 == 0)) &&
                           (!r.has_bias || r.bias_row) && 128 * r.ldb * 2 <= kIntMax &&
                           128 * r.ldc * 2 <= kIntMax && cdiv(r.N, 128) * r.batch <= kIntMax;
    // what the tall kernel needs: A and B as for `fast` (C is written element by element, so
    // its alignment does not matter) and a narrow B, as [N, K] or as [K, N] in 16-byte
    // column chunks
    const bool tall_ok = (r.align_a ? r.align_a : r.align) >= 16 && (r.align_b ? r.align_b : r.align) >= 16 &&
                         r.K % 8 == 0 && r.lda % 8 == 0 && r.ldb % 8 == 0 && r.N <= 128 &&
                         (r.layout == kNK || r.N % 8 == 0) &&
                         (!batched || (r.stride_a % 8 == 0 && r.stride_b % 8 == 0));
    if (skinny_ok && !skinny_tiles_enough && r.layout == kNK) {
      // B is [N, K] (a Linear weight): strips of W rows.  With at most half as many strips
      // as CUs and >= 700 KB to stream per workgroup (its W rows and A's 16-row blocks over
      // all of K), K is split so that ~256 workgroups run: a split costs a second launch
      // (~3 us) and saves streaming time in proportion (MI355X, fp16, W from HBM, unsplit vs
      // split: x[1, 14336] W[1024, 14336]^T 14.5 vs 10.5 us (4 ways), x[16, 14336] W[512,
      // 14336]^T 18.9 vs 10.9 (8), x[64, 8192] W[512, 8192]^T 20.6 vs 11.0 (8), x[64, 14336]
      // W[2048, 14336]^T 37.9 vs 25.6 (2)).  Below that the second launch outweighs what
      // it saves once W stays in the Infinity Cache between calls (x[64, 4096] W[1024,
      // 4096]^T, 655 KB: 12.9 vs 11.1 us from HBM but 9.9 vs 12.4 cached), and with 224
      // strips (x[64, 4096] W[14336, 4096]^T) 2 ways took 39.2 us against 29.3.
      p = skinny_nk_plan(r, 1, p.group_m);
      const int64_t chunk = std::min<int64_t>(r.batch, 65535);
      const int64_t wgs = cdiv(r.N, p.bn) * chunk, wgs64 = cdiv(r.N, 64) * chunk;
      if (2 * wgs <= kNumCUs && (int64_t)(p.bn + p.bm) * r.K * 2 >= 700000) {
        p = skinny_nk_plan(r, std::min<int64_t>(8, std::max<int64_t>(2, kNumCUs / wgs)), p.group_m);
      } else if (p.mb >= 2 && r.K >= 10240 && 2 * wgs64 <= kNumCUs) {
        // Long K with more than 16 rows of A over enough narrow strips: each 16-row strip
        // re-reads all of A from L2 (4x W's bytes at 64 rows), so 64-row strips with K split
        // to ~256 workgroups instead (MI355X, fp16, W from HBM: x[64, 14336] W[4096,
        // 14336]^T 40.9 -> 31.3 us, x[32, 14336] W[4096, 14336]^T 29.6 -> 25.7, x[64, 14336]
        // W[8192, 14336]^T 56.4 -> 50.8, x[48, 10240] W[4096, 10240]^T 28.3 -> 23.0; at K =
        // 8192 the unsplit narrow strips stay faster: x[64, 8192] W[4096, 8192]^T 22.7 vs 24.8)
        Plan q = skinny_nk_plan(r, std::max<int64_t>(2, kNumCUs / wgs64), p.group_m);
        if (q.splits > 1) {
          q.bn = 64;
          p = q;
        }
      }
    } else if (skinny_ok && !skinny_tiles_enough) {
      p.mb = (int)std::max<int64_t>(1, cdiv(r.M, 16));
      p.bm = 16 * p.mb;
      // Wide strips (128 columns: full 256-byte row segments, the faster HBM
      // pattern) with K split over workgroups until ~256 of them exist; the
      // splits need an fp32 workspace.  Narrow strips (32 columns, no split)
      // when there is no workspace or the wide grid would be much smaller.
      const int64_t chunk = std::min<int64_t>(r.batch, 65535);
      const int64_t strips = cdiv(r.N, 128);
      int64_t splits = 1;
      // (empty problems -- N or batch 0 -- launch nothing; keep the arithmetic defined)
      const int64_t wgs1 = std::max<int64_t>(1, strips * chunk);
      if (wgs1 < 192) splits = std::min<int64_t>(8, std::max<int64_t>(1, 256 / wgs1));
      splits = std::min<int64_t>(splits, std::max<int64_t>(1, r.K / 256));
      const int64_t need = splits > 1 ? splits * chunk * r.M * r.N * 4 : 0;
      const int64_t wide_wgs = strips * splits * chunk, narrow_wgs = cdiv(r.N, 32) * chunk;
      if (need <= r.ws_bytes && 2 * wide_wgs >= std::min<int64_t>(narrow_wgs, 256)) {
        p.kernel = kSkinnyWide;
        p.bn = 128;
        p.splits = (int)splits;
        p.ksplit = (int)(cdiv(cdiv(r.K, splits), 64) * 64);
        p.ws_bytes = need;
      } else {
        p.kernel = kSkinny;
        p.bn = 32;
      }
    } else if (stream_ok && cdiv(r.N, 128) * r.batch * cdiv(r.M, r.M <= 64 ? 64 : 128) >= 16 * kNumCUs) {
      // Short K over many columns with one A (a 1x1 convolution: weight x every image's
      // pixels): bound by streaming B in and C out, which persistent workgroups with
      // three tiles in flight do faster than one tile per workgroup once each has >= 16
      // tiles (MI355X, vs the 64x256 tile: 64 x 16384 x 128 x 64 images 64.0 vs 106.8
      // us, 64 x 1048576 x 128 60.5 vs 100.2, 64 x 16384 x 64 x 32 images 23.4 vs 38.2;
      // with 2 .. 8 tiles each it is up to 10 % slower).
      // (>= 16 tiles per workgroup: row blocks x column tiles over the 256 workgroups)
      p.kernel = r.M <= 64 ? kStream64x128 : kStream128x128;
      p.bm = r.M <= 64 ? 64 : 128;
      p.bn = 128;
      p.threads = r.M <= 64 ? 256 : 512;
    } else if (tall_ok && r.N <= 64 && r.M >= 1024 && r.K >= 1024 && cdiv(r.M, 128) * r.batch < kNumCUs &&
               (r.K <= 2048 ||
                (r.K <= 4096 && (r.M * r.batch >= 8192 || (r.layout == kNK && r.N <= 32))))) {
      // A narrow B (<= 64 columns) under fewer 128-row tiles than CUs: the tile kernels would
      // split K (or leave CUs idle) to fill the GPU; strips of A's rows over all of K stream
      // A once instead (MI355X, fp16, best strip vs the selector's tile128x128 (+ split):
      // 2048 x 64 x 2048 8.5 vs 10.8 us, 8192 x 64 x 2048 10.4 vs 16.1, 16384 x 64 x 2048
      // 16.6 vs 25.0, 16384 x 16 x 4096 27.7 vs 30.7, attention's P V over 8 x 2048 x 2048
      // with 64 columns 18.8 vs 25.7; measured slower from K = 8192, with 64 < N <= 128, or
      // at K = 4096 below 8192 rows -- except B as [N, K] with <= 32 rows, on one or two
      // 16-row blocks: 4096 x 16 x 4096 7.9 vs 10.8 us, 1024 x 32 x 4096 8.7 vs 9.4).  64-row strips once they give every CU one and K >=
      // 2048, else 32-row strips.
      p = tall_plan(r, cdiv(r.M, 64) * r.batch >= kNumCUs && r.K >= 2048 ? 64 : 32, p.group_m);
    } else if (tall_ok && r.N <= 64 && r.M >= 1024 && r.K >= 8192 && cdiv(r.M, 32) * r.batch <= 64 &&
               r.N % 4 == 0) {
      // ... and with long K over at most 64 strips of 32 rows, K split so that ~256
      // workgroups run (fp32 partials, a second launch sums them; MI355X, fp16, vs the
      // selector's tile128x128 split 16 ways: 1024 x 16 x 14336 9.9 vs 14.3 us, 1024 x 64 x
      // 14336 13.0 vs 15.5, 2048 x 8 x 14336 13.3 vs 16.4, 1024 x 64 x 8192 10.7 vs 11.6)
      p = tall_plan(r, 32, p.group_m, std::min<int64_t>(8, kNumCUs / (cdiv(r.M, 32) * r.batch)));
    } else if (fast && r.M <= 64 && r.K <= 1024 && cdiv(r.N, 256) * r.batch >= kNumCUs) {
      // Short-K products with few rows and many columns are HBM-bound; 64-row tiles
      // waste no MFMA rows and keep more loads in flight per CU (MI355X, 64x256 vs
      // 128x128: 64x1048576x128 103 vs 122 us, 32x131072x256 14.4 vs 17.3 us; at
      // K >= 2048 the 128x128 tile or the skinny kernel is faster).
      p.kernel = kTile64x256;
      p.bm = 64;
      p.bn = 256;
    } else if (fast) {
      // Tile and K split with the lowest modelled cost.  Splitting pays where the tiles
      // leave CUs idle and K is long (e.g. 256 x 4096 x 14336: 64 tiles of 128x128 for
      // 512 workgroup slots); K >= 2048, each split keeps >= 8 K steps, and needs the workspace for
      // its fp32 partials and N % 4 == 0.  Not for M <= 64: those products are bound by
      // streaming B, which a split does not shorten.
      const Candidate* best = &kTiles16[0];
      int64_t best_s = 1;
      double best_cost = -1.0;
      for (const Candidate& c : kTiles16) {
        const int64_t smax = (r.N % 4 == 0 && r.M > 64 && r.K >= 2048) ? std::min<int64_t>(16, r.K / 512) : 1;
        for (int64_t s = 1; s <= std::max<int64_t>(1, smax); ++s) {
          if (s > 1 && s * r.batch * r.M * r.N * 4 > r.ws_bytes) break;
          const double cost = split_cost(c, r.M, r.N, r.K, r.batch, s);
          if (best_cost < 0 || cost < best_cost) {
            best_cost = cost;
            best = &c;
            best_s = s;
          }
        }
      }
      p.kernel = best->id;
      p.bm = best->bm;
      p.bn = best->bn;
      if (best->id != kTile128x128) p.threads = 512;  // the 256-row tiles run 8 waves, 128x128 4
      if (best_s > 1) {
        p.splits = (int)best_s;
        p.ksplit = (int)(cdiv(cdiv(r.K, best_s), 64) * 64);
        p.ws_bytes = best_s * r.batch * r.M * r.N * 4;
      }
    } else {
      p.kernel = kGeneric16;
      p.bm = 64;
      p.bn = 64;
    }
    override16(r, fast, stream_ok, tall_ok, skinny_ok && r.layout == kNK, &p);
  }
  if (p.splits == 0) p.splits = 1;
  if (p.kernel == kSkinny || p.kernel == kSkinnyWide || p.kernel == kSkinnyNK || p.kernel == kStream64x128 ||
      p.kernel == kStream128x128) {
    // one grid column per column strip or tile: these kernels cover all of M themselves (the
    // streaming kernel in row blocks of bm)
    p.tiles_m = 1;
    p.tiles_n = (int)cdiv(r.N, p.bn) * (p.kernel == kSkinnyWide ? p.splits : 1);
  } else {
    p.tiles_m = (int)cdiv(r.M, p.bm);
    p.tiles_n = (int)cdiv(r.N, p.bn);
  }
  *plan = p;
  return CMPEXT3_OK;
}
}  // namespace

// Plans the request; when the only kernel that fits a 16-bit product is the
// element-wise generic one (rows not 16-byte aligned), and the product is large
// enough to pay for two copies, plans zero-padded, aligned copies of A and/or B in
// the workspace instead (K padded to a multiple of 8 with zeros, which adds
// exact zeros to every sum) and a tiled kernel on them.
static const F32Tile& f32_tile(KernelId id) {
  for (const F32Tile& c : kTiles32)
    if (c.id == id) return c;
  return kTiles32[0];
}

// fp32 operands whose rows are not 16-byte aligned run on the 4-byte DMA path; with a
// workspace, zero-padded copies (K, and N for B given as [K, N], rounded up to 4) let
// the 16-byte path run instead.  Taken when the model says the copies (read and write
// at ~4.5 TB/s, ~4.5 us per launch) cost at least 5 % less than the 4-byte path (the
// model is good to a few per cent here).  Measured on MI355X, padded vs direct:
// 2500 x 2501 x 2502 310 vs 344 us, 2049 x 2999 x 3001 377 vs 410 (both padded);
// 3001^3 492 vs 463 and cfg5 (4097 x 3001 x 2049; 96x64 loses 2.6 %) not padded.
static int plan_f32_padded(const Request& r, Plan* plan) {
  if (plan->dma16 || r.M == 0 || r.N == 0 || r.K == 0 || r.batch == 0) return CMPEXT3_OK;
  const int aa = r.align_a ? r.align_a : r.align, ab = r.align_b ? r.align_b : r.align;
  const bool kn = r.layout == kKN, batched = r.batch > 1;
  const int64_t kp = cdiv(r.K, 4) * 4, np = cdiv(r.N, 4) * 4;
  const bool pad_a = r.K % 4 != 0 || r.lda % 4 != 0 || aa < 16 || (batched && r.stride_a % 4 != 0);
  const bool pad_b = r.K % 4 != 0 || r.ldb % 4 != 0 || ab < 16 || (kn && r.N % 4 != 0) ||
                     (batched && r.stride_b % 4 != 0);
  Request q = r;
  q.K = kp;
  int64_t a_bytes = 0, b_bytes = 0;
  double copy_us = 0.0;
  if (pad_a) {
    const int64_t copies = (batched && r.stride_a != 0) ? r.batch : 1;
    q.lda = kp;
    q.stride_a = copies > 1 ? r.M * kp : 0;
    a_bytes = cdiv(r.M * kp * 4 * copies, 256) * 256;
    copy_us += 2.0 * (double)a_bytes / 4.5e6 + 4.5;
  }
  if (pad_b) {
    const int64_t copies = (batched && r.stride_b != 0) ? r.batch : 1;
    const int64_t rows = kn ? kp : r.N, cols = kn ? np : kp;
    q.ldb = cols;
    q.stride_b = copies > 1 ? rows * cols : 0;
    q.b_cols_padded = kn;
    b_bytes = cdiv(rows * cols * 4 * copies, 256) * 256;
    copy_us += 2.0 * (double)b_bytes / 4.5e6 + 4.5;
  }
  if (a_bytes + b_bytes > r.ws_bytes) return CMPEXT3_OK;
  q.align_a = pad_a ? 16 : aa;
  q.align_b = pad_b ? 16 : ab;
  q.align = std::min(q.align_a, q.align_b);
  q.ws_bytes = r.ws_bytes - a_bytes - b_bytes;
  Plan p2;
  if (make_plan_core(q, &p2) != CMPEXT3_OK || !p2.dma16) return CMPEXT3_OK;
  const double now = f32_cost(f32_tile(plan->kernel), r.M, r.N, r.K, r.batch, std::max(1, plan->splits), false);
  const double padded =
      copy_us + f32_cost(f32_tile(p2.kernel), r.M, r.N, kp, r.batch, std::max(1, p2.splits), true);
  if (padded >= 0.95 * now) return CMPEXT3_OK;
  p2.pad_a = pad_a;
  p2.pad_b = pad_b;
  p2.kp = kp;
  p2.lda_p = q.lda;
  p2.ldb_p = q.ldb;
  p2.stride_a_p = q.stride_a;
  p2.stride_b_p = q.stride_b;
  p2.pad_a_bytes = a_bytes;
  p2.pad_b_bytes = b_bytes;
  p2.ws_bytes += a_bytes + b_bytes;
  *plan = p2;
  return CMPEXT3_OK;
}

int make_plan(const Request& r, Plan* plan) {
  const int st = make_plan_core(r, plan);
  if (st == CMPEXT3_OK && r.dtype == kF32) return plan->forced ? st : plan_f32_padded(r, plan);
  if (st != CMPEXT3_OK || plan->kernel != kGeneric16 || plan->forced) return st;
  const double work = (double)r.M * (double)r.N * (double)r.K * (double)r.batch;
  const int aa = r.align_a ? r.align_a : r.align, ab = r.align_b ? r.align_b : r.align;
  const int ac = r.align_c ? r.align_c : r.align;
  if (work < (double)(1 << 24) || ac < 16) return st;
  const bool kn = r.layout == kKN, batched = r.batch > 1;
  const int64_t kp = cdiv(r.K, 8) * 8, np = cdiv(r.N, 8) * 8;
  const bool pad_a = r.K % 8 != 0 || r.lda % 8 != 0 || aa < 16 || (batched && r.stride_a % 8 != 0);
  const bool pad_b = r.K % 8 != 0 || r.ldb % 8 != 0 || ab < 16 || (kn && r.N % 8 != 0) ||
                     (batched && r.stride_b % 8 != 0);
  Request q = r;
  q.K = kp;
  int64_t a_bytes = 0, b_bytes = 0;
  if (pad_a) {
    q.lda = kp;
    q.stride_a = (batched && r.stride_a != 0) ? r.M * kp : 0;
    a_bytes = cdiv(r.M * kp * 2 * ((batched && r.stride_a != 0) ? r.batch : 1), 256) * 256;
  }
  if (pad_b) {
    const int64_t rows = kn ? kp : r.N, cols = kn ? np : kp;
    q.ldb = cols;
    q.stride_b = (batched && r.stride_b != 0) ? rows * cols : 0;
    q.b_cols_padded = kn;
    b_bytes = cdiv(rows * cols * 2 * ((batched && r.stride_b != 0) ? r.batch : 1), 256) * 256;
  }
  if (a_bytes + b_bytes > r.ws_bytes) return st;
  q.align_a = pad_a ? 16 : aa;
  q.align_b = pad_b ? 16 : ab;
  q.align = std::min(std::min(q.align_a, q.align_b), ac);
  q.ws_bytes = r.ws_bytes - a_bytes - b_bytes;
  Plan p2;
  if (make_plan_core(q, &p2) != CMPEXT3_OK || p2.kernel == kGeneric16) return st;
  p2.pad_a = pad_a;
  p2.pad_b = pad_b;
  p2.kp = kp;
  p2.lda_p = q.lda;
  p2.ldb_p = q.ldb;
  p2.stride_a_p = q.stride_a;
  p2.stride_b_p = q.stride_b;
  p2.pad_a_bytes = a_bytes;
  p2.pad_b_bytes = b_bytes;
  p2.ws_bytes += a_bytes + b_bytes;
  *plan = p2;
  return CMPEXT3_OK;
}


// Modelled time (us) of a 16-bit plan, for comparing a row split with the plan it would
// replace: the tile cost model above for the tiled kernels, and reading A and B and
// writing C once at ~5 TB/s for the HBM-bound ones; ~2 us per launch.
static double plan_us(const Request& r, const Plan& p) {
  for (const Candidate& c : kTiles16)
    if (c.id == p.kernel) return split_cost(c, r.M, r.N, r.K, r.batch, std::max(1, p.splits)) / kUnitsPerUs + 2.0;
  const double b_copies = (r.batch > 1 && r.stride_b != 0) ? (double)r.batch : 1.0;
  const double a_copies = (r.batch > 1 && r.stride_a != 0) ? (double)r.batch : 1.0;
  const double bytes = 2.0 * (a_copies * r.M * r.K + b_copies * r.K * r.N + (double)r.batch * r.M * r.N);
  return bytes / 5.0e6 + 3.0;
}

bool plan_row_split(const Request& r, const Plan& full, RowSplit* out) {
  if ((r.dtype != kF16 && r.dtype != kBF16) || full.forced || full.pad_a || full.pad_b || r.M <= 256 ||
      r.N == 0 || r.K == 0 || r.batch == 0)
    return false;
  const Candidate* fc = nullptr;
  for (const Candidate& c : kTiles16)
    if (c.id == full.kernel) fc = &c;
  if (fc == nullptr) return false;
  // Only a last round at most half full after at least one full round: a fuller last
  // round runs at a higher clock than the model assumes (fewer busy CUs under the same
  // power limit), and the split did not pay there (MI355X, fp16 2100 x 4096 x 4096: 171
  // tiles of 256x224 in one partial round 69.9 us, split into 2048 rows of 128x128 and 52
  // rows of skinny_wide 76.5 us).
  const int64_t slots = (int64_t)kNumCUs * fc->occ;
  const int64_t wgs = (int64_t)full.tiles_m * full.tiles_n * r.batch * std::max(1, full.splits);
  const int64_t rem = wgs % slots;
  if (wgs <= slots || rem == 0 || 2 * rem > slots) return false;
  // rows covered by whole rounds of the 256-row tiles (one workgroup per CU), and whole 256-row tiles
  int64_t cand[3] = {r.M / 256 * 256, 0, 0};
  for (int i = 0; i < 2; ++i) {
    const int64_t cols = cdiv(r.N, i == 0 ? 256 : 224) * r.batch;
    if (cols <= kNumCUs) {
      const int64_t rows = 256 * (kNumCUs / cols);
      cand[1 + i] = r.M / rows * rows;
    }
  }
  const double full_us = plan_us(r, full);
  double best = 0.92 * full_us;
  bool found = false;
  for (int64_t m_main : cand) {
    if (m_main <= 0 || m_main >= r.M) continue;
    Request a = r, b = r;
    a.M = m_main;
    b.M = r.M - m_main;
    // (the tail's A and C start m_main rows in: 16-byte aligned as the rows are, m_main
    // being a multiple of 256)
    Plan pa, pb;
    if (make_plan(a, &pa) != CMPEXT3_OK || make_plan(b, &pb) != CMPEXT3_OK) continue;
    if (pa.pad_a || pa.pad_b || pb.pad_a || pb.pad_b || pa.kernel == kGeneric16 || pb.kernel == kGeneric16) continue;
    const double us = plan_us(a, pa) + plan_us(b, pb);
    if (us < best) {
      best = us;
      out->m_main = m_main;
      out->main = pa;
      out->tail = pb;
      found = true;
    }
  }
  return found;
}

std::string describe(const Request& r, const Plan& p) {
  static const char* dt[] = {"f16", "bf16", "f32"};
  char buf[256];
  snprintf(buf, sizeof buf, "kernel=%s dtype=%s layout=%s tile=%dx%d grid=%dx%dx%lld threads=%d",
           kernel_name(p.kernel), dt[r.dtype], r.layout == kKN ? "KN" : "NK", p.bm, p.bn, p.tiles_m,
           p.tiles_n, (long long)r.batch, p.threads);
  std::string s(buf);
  if (p.kernel == kSkinny || p.kernel == kSkinnyWide || p.kernel == kSkinnyNK || p.kernel == kTall) {
    snprintf(buf, sizeof buf, " mb=%d", p.mb);
    s += buf;
  }
  if (p.kernel == kSkinnyWide || p.splits > 1) {
    snprintf(buf, sizeof buf, " splits=%d ksplit=%d workspace=%lld", p.splits, p.ksplit, (long long)p.ws_bytes);
    s += buf;
  }
  if (p.dma16) s += " dma16";
  if (p.pad_a || p.pad_b) {
    snprintf(buf, sizeof buf, " padded=%s%s kp=%lld workspace=%lld", p.pad_a ? "A" : "", p.pad_b ? "B" : "",
             (long long)p.kp, (long long)p.ws_bytes);
    s += buf;
  }
  return s;
}

}  // namespace cmpext3
