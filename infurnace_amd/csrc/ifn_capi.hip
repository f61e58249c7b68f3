// Status strings and ABI version of the C entry points declared in
// include/infurnace_amd.h.
#include "ifn_common.hpp"

extern "C" const char* ifn_status_string(int status) {
  switch (status) {
    case IFN_OK: return "ok";
    case IFN_ERR_INVALID_ARGUMENT: return "invalid argument";
    case IFN_ERR_UNSUPPORTED: return "unsupported shape (head_dim/group/block_size not compiled)";
    case IFN_ERR_ALIGNMENT: return "device pointer not 16-byte aligned";
    case IFN_ERR_WORKSPACE: return "workspace missing or too small";
    case IFN_ERR_HIP: return "HIP launch error";
    default: return "unknown status";
  }
}

extern "C" int ifn_abi_version(void) { return 1; }
