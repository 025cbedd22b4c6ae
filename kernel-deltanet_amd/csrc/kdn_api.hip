// Status text and ABI version of the Kernel-DeltaNet C ABI.
#include "kdn_internal.hpp"

extern "C" const char* kdn_strerror(int status) {
  switch (status) {
    case KDN_OK: return "ok";
    case KDN_ERR_INVALID_ARGUMENT: return "invalid argument (null pointer, bad size, stride or dtype tag)";
    case KDN_ERR_UNSUPPORTED: return "unsupported shape (d_k must be 64, D 512 for the scan, d_v in {16,32,64,128})";
    case KDN_ERR_WORKSPACE_TOO_SMALL: return "workspace smaller than kdn_scan_workspace_bytes()";
    case KDN_ERR_MISALIGNED: return "pointer or row stride not aligned for 16-byte vector access";
    case KDN_ERR_DEVICE: return "HIP launch error";
    case KDN_ERR_CAPACITY: return "state pool has no free slot";
    default: return "unknown kdn status";
  }
}

extern "C" int kdn_abi_version(void) { return (2 << 16) | 3; }
