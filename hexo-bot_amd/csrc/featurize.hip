// Position featurizer on the GPU: placement records -> support set, node
// order, neighbour table and the 15 feature planes, written straight into the
// padded forward inputs (the collate layout of batching.py:45-80).
//
// Semantics: build_support (packages/shrimp/python/shrimp/support.py:84-205)
// and build_features / window scan / opponent's last turn
// (packages/shrimp/python/shrimp/features.py:80-240), with the facts of
// features.py:54-77 derived from the records as the reference derives them
// for a decision state (side to move, phase and the turn's first stone from
// the record count unless given).
//
// One workgroup per position over an LDS window of wq x wr axial cells (at
// most 64 x 64, stored densely, q-major) around the stones' bounding box
// (margin max(R + 1, 5) on every side, so the whole support and every
// window-scan cell lies inside):
//   1. records -> bounding box (block reduction), window origin;
//   2. stones placed (colour, record id, distance 0);
//   3. multi-source BFS as R + 1 dilation steps over the window;
//   4. window scan: every (stone, axis, shift) window of one colour marks its
//      empty cells hot / win-now (LDS atomics on a per-cell flag word);
//      the opponent's last turn and the turn's first stone are flagged too;
//   5. node order [legal | stones | halo], each ascending by (q, r): the
//      window is stored q-major, so one block-wide scan of three counters
//      over the cells gives every node its row;
//   6. one pass over the nodes writes features, neighbour rows, coords, mask.
#include "capi.hpp"
#include "common.hpp"

namespace shrimp {

namespace {

constexpr int FZ_WIN = 64;                 // largest window side (cells)
constexpr int FZ_CELLS = FZ_WIN * FZ_WIN;  // 4096
constexpr int FZ_THREADS = 256;
constexpr int FZ_NF = 15;

// feature planes (constants.py:41-56)
enum : int {
  P_OWN_STONE = 0, P_OPP_STONE = 1, P_EMPTY = 2, P_LEGAL = 3, P_PHASE_SECOND = 4,
  P_FIRST_STONE = 5, P_PLAYER_COLOUR = 6, P_OWN_RECENCY = 7, P_OPP_RECENCY = 8,
  P_OPP_HOT = 9, P_OWN_HOT = 10, P_DIST = 11, P_OPP_LAST_TURN = 12, P_OPP_WIN = 13,
  P_OWN_WIN = 14
};
// per-cell flag bits
enum : unsigned {
  FL_OWN_HOT = 1u, FL_OPP_HOT = 2u, FL_OWN_WIN = 4u, FL_OPP_WIN = 8u, FL_FIRST = 16u,
  FL_OPP_LAST = 32u
};
constexpr int HOT_MIN_COUNT = 4, WIN_NOW_COUNT = 5, HOT_MIN_PLACEMENTS = 7, WINDOW_LEN = 6;
constexpr float DIST_SCALE = 8.0f;  // LEGAL_RADIUS, whatever the support radius (constants.py:62)
constexpr unsigned char DIST_NONE = 255, COLOUR_NONE = 255;

__constant__ int kDq[6] = {1, 0, -1, -1, 0, 1};  // DIRECTIONS (constants.py:20-27)
__constant__ int kDr[6] = {0, 1, 1, 0, -1, -1};
__constant__ int kAq[3] = {1, 0, 1};             // window axes Q, R, QR (features.py:47)
__constant__ int kAr[3] = {0, 1, -1};

// turn structure (features.py:80-93): record 0 opens, odd ordinals are first
// stones, even ordinals second stones; player 0 opens, then pairs alternate
// starting with player 1
SHRIMP_DEV int record_phase(int ordinal) { return ordinal == 0 ? 0 : (ordinal % 2 == 1 ? 1 : 2); }
SHRIMP_DEV int record_player(int ordinal) { return ordinal == 0 ? 0 : 1 - ((ordinal - 1) / 2) % 2; }

}  // namespace

__global__ __launch_bounds__(FZ_THREADS) void featurize_kernel(
    const int32_t* __restrict__ rec_qr, const uint8_t* __restrict__ rec_owner,
    const int32_t* __restrict__ rec_index, const int64_t* __restrict__ rec_off,
    const uint8_t* __restrict__ player_in, const uint8_t* __restrict__ phase_in, int radius,
    int Npad, float* __restrict__ feats, int32_t* __restrict__ nbr, uint8_t* __restrict__ mask,
    int32_t* __restrict__ coords, int32_t* __restrict__ counts, int32_t* __restrict__ status) {
  __shared__ unsigned char s_dist[FZ_CELLS];
  __shared__ unsigned char s_col[FZ_CELLS];
  __shared__ unsigned s_flag[FZ_CELLS];
  __shared__ short s_rec[FZ_CELLS];
  __shared__ short s_node[FZ_CELLS];
  __shared__ int s_red[4][FZ_THREADS / 64];
  __shared__ int s_scan[3][FZ_THREADS];
  __shared__ int s_tot[3];
  __shared__ int s_bad;

  const int b = blockIdx.x;
  const int t = threadIdx.x;
  const int64_t r0 = rec_off[b];
  const int nrec = (int)(rec_off[b + 1] - r0);
  const int player = player_in ? (int)player_in[b] : record_player(nrec);
  const int phase = phase_in ? (int)phase_in[b] : record_phase(nrec);
  const int reach = radius + 1;
  const int margin = max(reach, WINDOW_LEN - 1);
  const bool dump = feats != nullptr;
  float* fb = dump ? feats + (int64_t)b * Npad * FZ_NF : nullptr;
  int32_t* nb = dump ? nbr + (int64_t)b * Npad * 6 : nullptr;

  // rows [from, Npad) of this position: zero features, absent neighbours
  auto pad_rows = [&](int from) {
    if (!dump) return;
    for (int i = from * FZ_NF + t; i < Npad * FZ_NF; i += FZ_THREADS) fb[i] = 0.f;
    for (int i = from * 6 + t; i < Npad * 6; i += FZ_THREADS) nb[i] = Npad;
    for (int i = from + t; i < Npad; i += FZ_THREADS) {
      mask[(int64_t)b * Npad + i] = 0;
      coords[((int64_t)b * Npad + i) * 2] = 0;
      coords[((int64_t)b * Npad + i) * 2 + 1] = 0;
    }
  };

  if (nrec == 0) {
    // no stones: the origin (legal) and its 6 neighbours (halo) sorted by
    // (q, r), all at distance 0 (support.py:145-162)
    const int sq[7] = {0, -1, -1, 0, 0, 1, 1};
    const int sr[7] = {0, 0, 1, -1, 1, -1, 0};
    if (t == 0) {
      counts[b * 4 + 0] = 7;
      counts[b * 4 + 1] = 1;
      counts[b * 4 + 2] = 0;
      counts[b * 4 + 3] = 6;
      status[b] = Npad < 7 ? 3 : 0;
    }
    if (Npad < 7 || !dump) return;
    if (t < 7) {
      float f[FZ_NF];
#pragma unroll
      for (int p = 0; p < FZ_NF; ++p) f[p] = 0.f;
      f[P_EMPTY] = 1.f;
      f[P_LEGAL] = t == 0 ? 1.f : 0.f;
      f[P_PHASE_SECOND] = phase == 2 ? 1.f : 0.f;
      f[P_PLAYER_COLOUR] = player == 0 ? 1.f : 0.f;
#pragma unroll
      for (int p = 0; p < FZ_NF; ++p) fb[t * FZ_NF + p] = f[p];
      for (int k = 0; k < 6; ++k) {
        int j = Npad;
        for (int u = 0; u < 7; ++u)
          if (sq[u] == sq[t] + kDq[k] && sr[u] == sr[t] + kDr[k]) j = u;
        nb[t * 6 + k] = j;
      }
      mask[(int64_t)b * Npad + t] = 1;
      coords[((int64_t)b * Npad + t) * 2] = sq[t];
      coords[((int64_t)b * Npad + t) * 2 + 1] = sr[t];
    }
    pad_rows(7);
    return;
  }

  // ---- 1. bounding box ---------------------------------------------------------------
  int qmin = 1 << 30, qmax = -(1 << 30), rmin = 1 << 30, rmax = -(1 << 30);
  for (int i = t; i < nrec; i += FZ_THREADS) {
    const int q = rec_qr[(r0 + i) * 2], r = rec_qr[(r0 + i) * 2 + 1];
    qmin = min(qmin, q);
    qmax = max(qmax, q);
    rmin = min(rmin, r);
    rmax = max(rmax, r);
  }
  for (int m = 32; m >= 1; m >>= 1) {
    qmin = min(qmin, __shfl_xor(qmin, m, 64));
    qmax = max(qmax, __shfl_xor(qmax, m, 64));
    rmin = min(rmin, __shfl_xor(rmin, m, 64));
    rmax = max(rmax, __shfl_xor(rmax, m, 64));
  }
  if ((t & 63) == 0) {
    s_red[0][t >> 6] = qmin;
    s_red[1][t >> 6] = qmax;
    s_red[2][t >> 6] = rmin;
    s_red[3][t >> 6] = rmax;
  }
  __syncthreads();
  qmin = s_red[0][0], qmax = s_red[1][0], rmin = s_red[2][0], rmax = s_red[3][0];
  for (int w = 1; w < FZ_THREADS / 64; ++w) {
    qmin = min(qmin, s_red[0][w]);
    qmax = max(qmax, s_red[1][w]);
    rmin = min(rmin, s_red[2][w]);
    rmax = max(rmax, s_red[3][w]);
  }
  const int oq = qmin - margin, orr = rmin - margin;  // window origin
  if (qmax - qmin + 2 * margin + 1 > FZ_WIN || rmax - rmin + 2 * margin + 1 > FZ_WIN ||
      nrec > 32767) {
    if (t == 0) {
      status[b] = 2;  // the support does not fit the window
      counts[b * 4 + 0] = counts[b * 4 + 1] = counts[b * 4 + 2] = counts[b * 4 + 3] = 0;
    }
    pad_rows(0);
    return;
  }
  const int wq = qmax - qmin + 2 * margin + 1, wr = rmax - rmin + 2 * margin + 1;
  const int ncell = wq * wr;
  auto cell = [&](int q, int r) { return (q - oq) * wr + (r - orr); };
  for (int i = t; i < ncell; i += FZ_THREADS) {
    s_dist[i] = DIST_NONE;
    s_col[i] = COLOUR_NONE;
    s_flag[i] = 0u;
    s_rec[i] = -1;
    s_node[i] = -1;
  }
  __syncthreads();

  // ---- 2. stones -----------------------------------------------------------------------
  for (int i = t; i < nrec; i += FZ_THREADS) {
    const int c = cell(rec_qr[(r0 + i) * 2], rec_qr[(r0 + i) * 2 + 1]);
    s_col[c] = rec_owner[r0 + i] ? 1 : 0;
    s_dist[c] = 0;
    s_rec[c] = (short)i;
  }
  __syncthreads();

  // ---- 3. BFS distances: dilation steps 1 .. R + 1 ---------------------------------------
  for (int d = 1; d <= reach; ++d) {
    for (int c = t; c < ncell; c += FZ_THREADS) {
      if (s_dist[c] != DIST_NONE) continue;
      const int cq = c / wr, cr = c - cq * wr;
      bool hit = false;
#pragma unroll
      for (int k = 0; k < 6; ++k) {
        const int nq = cq + kDq[k], nr = cr + kDr[k];
        if (nq >= 0 && nq < wq && nr >= 0 && nr < wr && s_dist[nq * wr + nr] == (unsigned char)(d - 1))
          hit = true;
      }
      if (hit) s_dist[c] = (unsigned char)d;
    }
    __syncthreads();
  }

  // ---- 4. window scan (features.py:99-159), first stone, opponent's last turn -----------
  const bool hot_enabled = nrec >= HOT_MIN_PLACEMENTS;
  for (int w = t; w < nrec * 3 * WINDOW_LEN; w += FZ_THREADS) {
    const int i = w / (3 * WINDOW_LEN), rem = w - i * 3 * WINDOW_LEN;
    const int ax = rem / WINDOW_LEN, shift = rem - ax * WINDOW_LEN;
    const int q0 = rec_qr[(r0 + i) * 2] - shift * kAq[ax];
    const int rr0 = rec_qr[(r0 + i) * 2 + 1] - shift * kAr[ax];
    int cnt[2] = {0, 0};
#pragma unroll
    for (int k = 0; k < WINDOW_LEN; ++k) {
      const unsigned char col = s_col[cell(q0 + k * kAq[ax], rr0 + k * kAr[ax])];
      if (col != COLOUR_NONE) ++cnt[col];
    }
    if (cnt[0] && cnt[1]) continue;
    const int owner = cnt[0] ? 0 : 1;
    const bool own = owner == player;
    const int total = cnt[0] + cnt[1];
    unsigned fl = 0u;
    if (total == WIN_NOW_COUNT) fl |= own ? FL_OWN_WIN : FL_OPP_WIN;
    if (total >= HOT_MIN_COUNT && hot_enabled) fl |= own ? FL_OWN_HOT : FL_OPP_HOT;
    if (!fl) continue;
#pragma unroll
    for (int k = 0; k < WINDOW_LEN; ++k) {
      const int c = cell(q0 + k * kAq[ax], rr0 + k * kAr[ax]);
      if (s_col[c] == COLOUR_NONE) atomicOr(&s_flag[c], fl);
    }
  }
  if (t == 0) {
    // the turn's first stone: the last record while the second stone is due
    if (phase == 2) {
      const int64_t li = r0 + nrec - 1;
      atomicOr(&s_flag[cell(rec_qr[li * 2], rec_qr[li * 2 + 1])], FL_FIRST);
    }
    // the opponent's newest full turn (features.py:213-233)
    const int opponent = 1 - player;
    for (int o = nrec - 1; o >= 0; --o) {
      if (record_player(o) != opponent) continue;
      const int ph = record_phase(o);
      if (ph == 2) {
        atomicOr(&s_flag[cell(rec_qr[(r0 + o - 1) * 2], rec_qr[(r0 + o - 1) * 2 + 1])], FL_OPP_LAST);
        atomicOr(&s_flag[cell(rec_qr[(r0 + o) * 2], rec_qr[(r0 + o) * 2 + 1])], FL_OPP_LAST);
        break;
      }
      if (ph == 0) {
        atomicOr(&s_flag[cell(rec_qr[(r0 + o) * 2], rec_qr[(r0 + o) * 2 + 1])], FL_OPP_LAST);
        break;
      }
    }
  }
  __syncthreads();

  // ---- 5. node order: legal | stones | halo, each q-major over the window ---------------
  // category of a cell: 0 legal (1 <= d <= R), 1 stone (d = 0), 2 halo (d = R + 1)
  auto category = [&](int c) -> int {
    const unsigned char d = s_dist[c];
    if (d == DIST_NONE) return -1;
    if (d == 0) return 1;
    return d <= radius ? 0 : 2;
  };
  int loc[3] = {0, 0, 0};
  const int cpt = (ncell + FZ_THREADS - 1) / FZ_THREADS;  // cells per thread, contiguous
  const int c_begin = min(t * cpt, ncell), c_end = min(c_begin + cpt, ncell);
  for (int c = c_begin; c < c_end; ++c) {
    const int k = category(c);
    if (k >= 0) ++loc[k];
  }
#pragma unroll
  for (int k = 0; k < 3; ++k) s_scan[k][t] = loc[k];
  __syncthreads();
  // inclusive Hillis-Steele scan of the three counters over the threads
  for (int off = 1; off < FZ_THREADS; off <<= 1) {
    int v[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) v[k] = t >= off ? s_scan[k][t - off] : 0;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 3; ++k) s_scan[k][t] += v[k];
    __syncthreads();
  }
  if (t == FZ_THREADS - 1) {
#pragma unroll
    for (int k = 0; k < 3; ++k) s_tot[k] = s_scan[k][t];
  }
  __syncthreads();
  const int n_legal = s_tot[0], n_stone = s_tot[1], n_halo = s_tot[2];
  const int n = n_legal + n_stone + n_halo;
  {
    const int base[3] = {0, n_legal, n_legal + n_stone};
    int rank[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) rank[k] = base[k] + s_scan[k][t] - loc[k];
    for (int c = c_begin; c < c_end; ++c) {
      const int k = category(c);
      if (k >= 0) s_node[c] = (short)(rank[k]++);
    }
  }
  if (t == 0) {
    counts[b * 4 + 0] = n;
    counts[b * 4 + 1] = n_legal;
    counts[b * 4 + 2] = n_stone;
    counts[b * 4 + 3] = n_halo;
    s_bad = n > Npad || n > 32767;
    status[b] = s_bad ? 3 : 0;  // 3: more nodes than Npad (rows past it are dropped)
  }
  __syncthreads();
  if (!dump) return;

  // ---- 6. emit the nodes -----------------------------------------------------------------
  const float colour_plane = player == 0 ? 1.f : 0.f;
  const float phase_plane = phase == 2 ? 1.f : 0.f;
  for (int c = t; c < ncell; c += FZ_THREADS) {
    const int row = s_node[c];
    if (row < 0 || row >= Npad) continue;
    const int cq = c / wr, cr = c - cq * wr;
    float f[FZ_NF];
#pragma unroll
    for (int p = 0; p < FZ_NF; ++p) f[p] = 0.f;
    const unsigned char col = s_col[c];
    if (col != COLOUR_NONE) {
      const int ri = s_rec[c];
      const bool own = col == player;
      const int placed = rec_index ? rec_index[r0 + ri] : ri;
      // 1 / (1 + placements since), rounded from double as the reference does
      const float rec = (float)(1.0 / (1.0 + (double)(nrec - placed)));
      f[own ? P_OWN_STONE : P_OPP_STONE] = 1.f;
      f[own ? P_OWN_RECENCY : P_OPP_RECENCY] = rec;
    }
    f[P_EMPTY] = 1.f - f[P_OWN_STONE] - f[P_OPP_STONE];
    f[P_LEGAL] = row < n_legal ? 1.f : 0.f;
    f[P_PHASE_SECOND] = phase_plane;
    f[P_PLAYER_COLOUR] = colour_plane;
    const unsigned fl = s_flag[c];
    if (phase == 2 && (fl & FL_FIRST)) f[P_FIRST_STONE] = 1.f;
    if (fl & FL_OPP_HOT) f[P_OPP_HOT] = 1.f;
    if (fl & FL_OWN_HOT) f[P_OWN_HOT] = 1.f;
    if (fl & FL_OPP_WIN) f[P_OPP_WIN] = 1.f;
    if (fl & FL_OWN_WIN) f[P_OWN_WIN] = 1.f;
    if (fl & FL_OPP_LAST) f[P_OPP_LAST_TURN] = 1.f;
    f[P_DIST] = (float)s_dist[c] / DIST_SCALE;
#pragma unroll
    for (int p = 0; p < FZ_NF; ++p) fb[row * FZ_NF + p] = f[p];
#pragma unroll
    for (int k = 0; k < 6; ++k) {
      const int nq = cq + kDq[k], nr = cr + kDr[k];
      int j = Npad;
      if (nq >= 0 && nq < wq && nr >= 0 && nr < wr) {
        const int v = s_node[nq * wr + nr];
        if (v >= 0 && v < Npad) j = v;
      }
      nb[row * 6 + k] = j;
    }
    mask[(int64_t)b * Npad + row] = 1;
    coords[((int64_t)b * Npad + row) * 2] = cq + oq;
    coords[((int64_t)b * Npad + row) * 2 + 1] = cr + orr;
  }
  pad_rows(min(n, Npad));
}

}  // namespace shrimp

using namespace shrimp;

extern "C" int shrimp_featurize(const int32_t* rec_qr, const uint8_t* rec_owner,
                                const int32_t* rec_index, const int64_t* rec_offsets,
                                const uint8_t* player, const uint8_t* phase, int B, int radius,
                                int Npad, float* feats, int32_t* nbr, uint8_t* mask,
                                int32_t* coords, int32_t* counts, int32_t* status, void* stream) {
  SHRIMP_REQUIRE(B >= 0, "featurize: B %d", B);
  if (B == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(rec_offsets && counts && status, "featurize: null pointer");
  SHRIMP_REQUIRE(radius >= 1 && radius <= 24, "featurize: radius %d outside [1, 24]", radius);
  SHRIMP_REQUIRE(!feats || (nbr && mask && coords && Npad >= 1 && Npad <= 32767),
                 "featurize: outputs need nbr, mask, coords and 1 <= Npad <= 32767");
  hipLaunchKernelGGL(featurize_kernel, dim3(B), dim3(FZ_THREADS), 0, as_stream(stream), rec_qr,
                     rec_owner, rec_index, rec_offsets, player, phase, radius, Npad, feats, nbr,
                     mask, coords, counts, status);
  return check_launch("featurize");
}
