// lds_layout.h -- placement of 16-byte chunks in the LDS tiles of the
// gfx950 attention kernels (shared with the host-side bank-conflict check,
// tests/cpp/check_lds_banks.cpp).
#pragma once
#include "mask.h"  // CHIA_HD

namespace chia {

// Swizzled 16-byte slot of chunk c of row r in an LDS tile (an XOR mask per
// row, so the map is its own inverse).  The LDS has 64 four-byte banks;
// ds_read_b128 serves 16 lanes per pass, ds_read_b64(_tr_b16) 32 lanes.
//   row_swz: the mask of tiles read by rows (16 lanes = 16 consecutive rows,
//     one logical chunk) AND transposed (32 lanes = 4 consecutive rows x 4
//     logical chunks), both without bank conflicts.  Rows of 128 bytes (D 64)
//     alternate between the two bank halves, so the even rows of 16 need 8
//     distinct masks (bits 1-3 of r), and rows r, r + 2 of a transposed group
//     differ in mask bit 2 (bit 1 of r).  Rows of 256 bytes (D 128) span all
//     banks: the 16 rows need 16 distinct masks, and the 4 rows of a
//     transposed group distinct bits 2-3 (r & 3).
//   k_slot: the forward's K tile (row reads) and every backward tile.
//   v_slot: the forward's V tile (transposed reads only).
// The mask is XOR-linear in the row's bits, which the transposed reads use:
// row + 8 flips it by row_swz(8), and row + 16 c leaves it unchanged.
template <int D>
CHIA_HD int row_swz(int r) {
  return D == 64 ? (((r >> 1) & 1) << 2) | (((r >> 2) & 1) << 1) | ((r >> 3) & 1) : ((r & 3) << 2) | ((r >> 2) & 3);
}
template <int D>
CHIA_HD int k_slot(int r, int c) {
  return c ^ row_swz<D>(r);
}
template <int D>
CHIA_HD int v_slot(int r, int c) {
  return c ^ ((D == 64 ? 2 : 4) * (r & 3));
}

}  // namespace chia
