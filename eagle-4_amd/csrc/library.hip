// Library introspection of the eagle4_amd C ABI: version string and the argument-struct sizes the host binding checks.

#include "common.h"

extern "C" const char* eagle4_version(void) { return "eagle4_amd 0.1.0 gfx950"; }

extern "C" int64_t eagle4_args_size(int which) {
  switch (which) {
    case 0: return sizeof(eagle4_stage_tree_args);
    case 1: return sizeof(eagle4_ancestors_args);
    case 2: return sizeof(eagle4_tail_words_args);
    case 3: return sizeof(eagle4_conv_args);
    case 4: return sizeof(eagle4_gdn_args);
    case 5: return sizeof(eagle4_records_args);
    case 6: return sizeof(eagle4_records_commit_args);
    case 7: return sizeof(eagle4_attn_args);
    case 8: return sizeof(eagle4_argmax_args);
    case 9: return sizeof(eagle4_accept_tree_args);
    case 10: return sizeof(eagle4_accept_tail_args);
    case 11: return sizeof(eagle4_compact_rows_args);
    case 12: return sizeof(eagle4_state_commit_args);
    case 13: return sizeof(eagle4_compact_kv_args);
    case 14: return sizeof(eagle4_chainize_args);
    case 15: return sizeof(eagle4_row_attn_args);
    case 16: return sizeof(eagle4_mamba2_args);
    default: return -1;
  }
}
