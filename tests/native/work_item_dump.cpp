// Host-side dump of the attention kernels' workgroup -> work-item mapping
// (work_item in attn_common.h) for tests/test_work_item.py:
//   work_item_dump groups m_blocks group ilv  ->  one line per workgroup: "bid item"
//   work_item_dump --ilv max_seqlen_k head_dim  ->  interleave_groups
#include <cstdio>
#include <cstdlib>

#include "attn_common.h"

int main(int argc, char** argv) {
  if (argc == 4 && argv[1][0] == '-') {
    printf("%d\n", tmx::interleave_groups(atol(argv[2]), atoi(argv[3])));
    return 0;
  }
  if (argc != 5) return 2;
  const long groups = atol(argv[1]), m_blocks = atol(argv[2]), group = atol(argv[3]);
  const int ilv = atoi(argv[4]);
  const long ipg = m_blocks * group;
  const long total = groups * ipg;
  const long grid = 8 * tmx::work_items_per_xcd(groups, ipg);
  for (long bid = 0; bid < grid; ++bid)
    printf("%ld %d\n", bid, tmx::work_item((int)bid, (int)total, (int)ipg, ilv));
  return 0;
}
