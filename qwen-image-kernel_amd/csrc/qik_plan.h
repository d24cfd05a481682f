// Workgroup -> work assignment of the attention kernel, shared by the kernel
// and the host (launch geometry, workspace size, the work-map export).
//
// A work item is one row block (BM query rows of one (b, h)), numbered
// (b, h)-major with the heaviest row block of a head first.  Workgroups are
// dealt to the device's nx XCDs round-robin (XCD = blockIdx % nx; nx = 8 on
// MI355X, the hardware's dealing order measured there), so XCD x runs the
// workgroups x, x+nx, ...; each XCD gets a contiguous run of items (per + 1
// on the first `rem` XCDs, per on the rest) so that a head's K/V stays in one
// L2.  Coverage does not depend on that dealing order: the plan hands every
// item to exactly one queue position whatever nx is, so a device that deals
// workgroups differently (or reports another XCD count) only loses locality.
//
// An XCD holds `sx` workgroups at once.  Items that fill whole rounds of sx
// run as one unit each; each item of the last, partly filled round is split
// over its KV tiles into two pieces: a big one (the first seven tenths of its
// tiles) and a small one (the rest).  The order lists the big pieces of all
// left-over items first, then the small ones.  The launch with a workspace
// runs sx workgroups per XCD that pull the XCD's units from a queue in this
// order.  The two workgroups of a CU progress at different rates (the older
// one's waves win issue arbitration), so the slots of the last whole round
// free up in two waves: the first takes the big pieces, the second the small
// ones, and both finish about together (measured on MI355X: 0.6 to 0.75 of
// the tiles for the big piece are all within 1%), where equal halves leave
// the early slot idle while the late one finishes.  When an XCD has no whole
// round and every piece gets a slot of its own (a launch smaller than the
// device), all pieces start together and the launch lasts as long as the
// biggest: then the pieces are equal halves.  The two pieces of an item combine
// their partial softmax states through the workspace slots of its group.
//
// plan_work(pl, loc * nx + x) is the unit at queue position loc of XCD x;
// without a workspace the same function maps workgroup bid = loc * nx + x.

#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define QIK_HD __host__ __device__
#else
#define QIK_HD
#endif

namespace qik {

constexpr int NXCD = 8;        // XCDs of an MI355X (the plan's default)
constexpr int NXCD_MAX = 32;   // largest XCD count a plan takes (control-word layout)
constexpr int MAX_PIECES = 2;

struct WorkPlan {
  int nx;                // XCDs the workgroups are dealt to (1 .. NXCD_MAX)
  int nmb;               // row blocks per (b, h)
  int per, rem;          // items per XCD: per + 1 on XCDs x < rem, per on the others
  int full_lo, full_hi;  // items an XCD runs whole when it has per / per + 1 items
  int ns;                // pieces per split item (1: nothing is split)
  int wpx;               // positions per XCD: the workgroups of a launch without a
                         // workspace (grid nx * wpx), or the queue length of one
                         // with (grid nx * min(sx, wpx))
  int mb_major;          // 1: an XCD's items are whole heads, walked rank-major in pairs of heads
  int ngroups;           // split items (workspace slot groups of ns slots)
  int even;              // 1: the two pieces are equal halves, else 7/10 and 3/10
};

struct Work {
  int item;   // row block, or -1 for a workgroup with no work (grid padding)
  int piece;  // 0 .. ns-1 for a split item, 0 otherwise
  int group;  // workspace slot group of a split item, -1 otherwise
};

// Items of an XCD with q items that run whole when it holds sx workgroups.
QIK_HD inline int plan_full(int q, int sx) { return q >= sx ? sx * (q / sx) : 0; }

// Pieces per split item: two (see above).
inline int plan_pieces(int r) { return r > 0 ? MAX_PIECES : 1; }

// n items, nmb per (b, h); `split` = 0 runs every item whole.  `ragged`: the
// items of a head differ in weight (per-row causal lengths), so an XCD that
// holds whole heads walks them rank-major, two heads at a time (the heaviest
// row block of both heads first, the light ones last; then the next pair; an
// odd last head alone, heaviest first), so the split tail holds light row
// blocks while at most two heads' K/V are in flight in its L2 (measured on
// MI355X: three heads rank-major fetch 1.4x the bytes at the same time, one
// head at a time is 8% slower); with equal items it keeps them head-major.
inline WorkPlan make_plan(int n, int nmb, int sx, int split, int ragged = 1, int nx = NXCD) {
  WorkPlan pl;
  if (nx < 1) nx = 1;
  if (nx > NXCD_MAX) nx = NXCD_MAX;
  pl.nx = nx;
  pl.nmb = nmb;
  pl.per = n / nx;
  pl.rem = n % nx;
  if (sx < 1) sx = 1;
  if (split) {
    pl.full_lo = plan_full(pl.per, sx);
    pl.full_hi = plan_full(pl.per + 1, sx);
  } else {
    pl.full_lo = pl.per;
    pl.full_hi = pl.per + 1;
  }
  const int r_lo = pl.per - pl.full_lo, r_hi = pl.per + 1 - pl.full_hi;
  const int r_max = (pl.rem > 0 && r_hi > r_lo) ? r_hi : r_lo;
  pl.ns = plan_pieces(r_max);
  const int w_lo = pl.full_lo + pl.ns * r_lo;
  const int w_hi = pl.rem > 0 ? pl.full_hi + pl.ns * r_hi : 0;
  pl.wpx = w_lo > w_hi ? w_lo : w_hi;
  pl.ngroups = pl.rem * r_hi + (nx - pl.rem) * r_lo;
  pl.even = (pl.ns > 1 && pl.full_lo == 0 && pl.full_hi == 0 && pl.wpx <= sx) ? 1 : 0;
  pl.mb_major = (split && ragged && pl.rem == 0 && nmb > 0 && pl.per % nmb == 0) ? 1 : 0;
  return pl;
}

QIK_HD inline Work plan_work(const WorkPlan& pl, int bid) {
  const int x = bid % pl.nx, loc = bid / pl.nx;
  const int big = x < pl.rem ? 1 : 0;
  const int q = pl.per + big;
  const int full = big ? pl.full_hi : pl.full_lo;
  const int r = q - full;
  Work w;
  w.item = -1;
  w.piece = 0;
  w.group = -1;
  if (loc >= full + pl.ns * r) return w;
  int k = loc;
  if (loc >= full) {
    // left-over item t % r, piece t / r: every item's first piece, then every
    // item's second piece
    const int t = loc - full;
    const int nbig = x < pl.rem ? x : pl.rem;
    k = full + t % r;
    w.piece = t / r;
    w.group = nbig * (pl.per + 1 - pl.full_hi) + (x - nbig) * (pl.per - pl.full_lo) + t % r;
  }
  const int v0 = x * pl.per + (x < pl.rem ? x : pl.rem);
  if (pl.mb_major) {
    // rank-major over pairs of the XCD's heads, one pair after the other (an
    // odd last head alone): the heaviest row blocks of a pair first, the
    // lightest ones of the last pair (or head), and so the split tail, last
    const int heads = q / pl.nmb;
    const int g = k / (2 * pl.nmb);
    const int gh = (2 * g + 2 <= heads) ? 2 : 1;
    const int j = k - g * 2 * pl.nmb;
    w.item = v0 + (2 * g + j % gh) * pl.nmb + j / gh;
  } else {
    w.item = v0 + k;
  }
  return w;
}

}  // namespace qik
