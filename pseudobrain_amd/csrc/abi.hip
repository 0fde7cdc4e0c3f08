// Version and status text of the pbgdn C ABI.
#include "pbgdn.h"

extern "C" int pbgdn_abi_version(void) { return PBGDN_ABI_VERSION; }

extern "C" const char *pbgdn_status_string(int status) {
  switch (status) {
    case PBGDN_OK: return "ok";
    case PBGDN_ERR_INVALID_ARGUMENT: return "invalid argument (null pointer, size or dtype code)";
    case PBGDN_ERR_UNSUPPORTED: return "unsupported shape (head width, chunk or grid size)";
    case PBGDN_ERR_LAUNCH: return "HIP kernel launch failed";
    case PBGDN_ERR_SCRATCH:
      return "the call needs more workspace than the no-allocation entry point's scratch "
             "(PBGDN_NOALLOC_SCRATCH_BYTES) holds";
    default: return "unknown pbgdn status";
  }
}
