// GDN records contract on gfx950 (kernels/gdn_tree_records.py): replay records and the accepted-path commit.
#include "common.h"

extern "C" int eagle4_gdn_tree_records_update(const eagle4_records_args* a, void* stream) {
  (void)a;
  (void)stream;
  return EAGLE4_NOT_COVERED;
}

extern "C" int eagle4_gdn_tree_records_commit(const eagle4_records_commit_args* a, void* stream) {
  (void)a;
  (void)stream;
  return EAGLE4_NOT_COVERED;
}
