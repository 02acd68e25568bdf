// Work split of the one-token decode kernel (moe_decode1.hip) between its
// workgroups, shared by the kernel, its host-side shape check and a CPU test
// (plain C++: the test compiles this header with g++).
//
// G workgroups (one per CU), U unique experts, Tk = I / 32 intermediate
// column tiles, units = H / 32 output column units:
//   items   workgroups [0, U*Tk): one (expert, column tile) each;
//   whole   workgroups [U*Tk, U*Tk + n_whole): one output unit each;
//   folded  output units [n_whole, units): no workgroup of their own; item f
//           (f < n_left) sums folded unit n_whole + f from every item's
//           partial sums, so every folded unit needs an item: n_left <= U*Tk.
#pragma once

#if defined(__HIPCC__)
#define GI_D1_HD __host__ __device__
#else
#define GI_D1_HD
#endif

namespace gi {
namespace d1 {

struct Split {
  int n_items;  // item workgroups
  int n_whole;  // unit workgroups
  int n_left;   // folded units
};

GI_D1_HD inline Split split(int G, int U, int Tk, int units) {
  Split s;
  s.n_items = U * Tk;
  s.n_whole = units < G - s.n_items ? units : G - s.n_items;
  s.n_left = units - s.n_whole;
  return s;
}

// True when every U in [1, umax] gives a split the kernel can run (U = 0 has
// its own branch).  n_left = max(0, units - G + U*Tk) grows with U, so the
// limits are checked at umax; n_left <= U*Tk for every U >= 1 holds exactly
// when units <= G.
GI_D1_HD inline bool split_ok(int G, int umax, int Tk, int units, int max_left) {
  if (G < 1 || umax < 1 || Tk < 1 || units < 1) return false;
  if (umax * Tk > G) return false;  // every item has a workgroup
  if (units > G) return false;      // folded units never outnumber the items
  const Split s = split(G, umax, Tk, units);
  return s.n_left <= max_left && s.n_left <= s.n_whole;
}

}  // namespace d1
}  // namespace gi
