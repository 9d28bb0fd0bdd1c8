// prefill.hip -- placeholder until the MFMA kernel lands.
#include "fat_common.h"
extern "C" size_t fat_prefill_workspace_bytes(int32_t, int32_t, int32_t) { return 0; }
extern "C" int fat_prefill_varlen(const fat_prefill_args*, void*) {
  fat_host::set_error("fat_prefill_varlen: not built yet");
  return FAT_E_UNSUPPORTED;
}
