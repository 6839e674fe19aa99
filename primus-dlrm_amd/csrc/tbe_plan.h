// Host/device metadata of a pdm_tbe_plan, shared by the pooled forward and
// the fused backward.
#pragma once

#include <vector>

#include "pdm_common.h"

namespace pdm {

// Per slot (one pooled output), read by the forward kernels.
struct TbeMeta {
  int64_t rows;
  int64_t w_off;  // byte offset of row 0 inside the weights buffer
  int32_t row_bytes;
  int32_t out_col;
  int32_t pooling;
  int32_t dim;
};

// Slots sharing (dtype, dim), launched together by the forward.
struct TbeGroup {
  int32_t dtype;
  int32_t dim;
  int32_t row_bytes_all;  // common row stride, -1 if tables differ
  int32_t first;          // index into the grouped table list
  int32_t count;
  int32_t out_col_align;  // alignment (elements) of all out_offsets
  int32_t table_base;     // first table if the group's tables are consecutive, else -1
};

// Per slot, read by the backward's linearisation: the slot's table in the
// row space and where its bag gradients sit in grad_out.
struct BwdSlot {
  int64_t rows;
  int64_t row_off;  // row-space id of row 0 of the slot's table
  int32_t out_col;
  int32_t pooling;
};

// A distinct table (slots reading the same rows share one).
struct BwdTable {
  int64_t row_off;  // row-space id of row 0
  int64_t w_elem;   // fp32 element index of row 0 in the weights buffer
  int64_t s_off;    // index of row 0's entry in the row-wise optimizer state
};

// The distinct tables of one forward group occupy the contiguous row-space
// range [row_lo, row_hi); their BwdTable entries are
// d_bwd_tables[first_table, first_table + num_tables), sorted by row_off.
struct BwdGroup {
  int32_t dim;
  int32_t dtype;
  int32_t first_table;
  int32_t num_tables;
  int32_t dense_rows;  // every table of the group has row_bytes == 4 * dim
  int32_t reserved;
  int64_t row_lo;
  int64_t row_hi;
  int64_t w_delta;  // w_elem - row_off * dim, common to the group's tables; INT64_MIN if they differ
  int64_t s_delta;  // s_off - row_off, common to the group's tables; INT64_MIN if they differ
};

// Sets each group's s_delta from bwd_tables (after state offsets change).
inline void refresh_state_deltas(std::vector<BwdGroup>& groups, const std::vector<BwdTable>& tabs) {
  for (auto& g : groups) {
    g.s_delta = INT64_MIN;
    for (int i = 0; i < g.num_tables; ++i) {
      const BwdTable& t = tabs[g.first_table + i];
      const int64_t d = t.s_off - t.row_off;
      if (i == 0) g.s_delta = d;
      else if (d != g.s_delta) {
        g.s_delta = INT64_MIN;
        break;
      }
    }
  }
}

}  // namespace pdm

struct pdm_tbe_plan_s {
  int device = 0;
  std::vector<pdm_table_desc> tables;
  std::vector<pdm::TbeGroup> groups;
  pdm::TbeMeta* d_meta = nullptr;
  int32_t* d_group_tables = nullptr;
  int64_t total_dim = 0;
  // row space of the distinct tables (backward and optimizer state layout)
  std::vector<int64_t> slot_row_off;
  std::vector<int32_t> slot_table;  // index into bwd_tables of the slot's table (-1: no rows)
  std::vector<pdm::BwdTable> bwd_tables;
  std::vector<pdm::BwdGroup> bwd_groups;
  int64_t total_rows = 0;
  pdm::BwdSlot* d_bwd_slots = nullptr;
  pdm::BwdTable* d_bwd_tables = nullptr;
  ~pdm_tbe_plan_s();
};
