// The work-item bounds check of the attention kernels (work_item_fits in
// hexkv_common.h), compiled for the host so its arithmetic can be tested on
// the CPU with extreme item values.
#include "hexkv_common.h"

extern "C" int emu_item_fits(int row, int head_group, int part, int parts, int first, int count, int len, int rows,
                             int n_groups, int max_parts, int max_seqlen) {
  hexkv_work_item it{row, head_group, part, parts, first, count, len, 0};  // heads 0: any size
  return hexkv::work_item_fits(it, rows, n_groups, max_parts, max_seqlen) ? 1 : 0;
}
