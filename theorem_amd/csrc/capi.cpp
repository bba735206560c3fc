// Host-side entry points of libtheorem_mi355x.so that launch nothing.
#include "../../include/theorem_mi355x.h"

extern "C" int thm_abi_version(void) { return THM_ABI_VERSION; }

extern "C" const char* thm_status_string(int status) {
  switch (status) {
    case THM_OK: return "ok";
    case THM_ERR_NULL_POINTER: return "a required pointer is NULL";
    case THM_ERR_BAD_SHAPE: return "invalid shape (negative, zero, overflowing, or T not a multiple of the chunk size)";
    case THM_ERR_BAD_DTYPE: return "unsupported dtype code";
    case THM_ERR_UNSUPPORTED: return "size not supported by this build (K, V in {64,128}; conv width 1..8)";
    case THM_ERR_MISALIGNED: return "pointer not aligned to its element size";
    case THM_ERR_BAD_ARGUMENT: return "invalid flag, activation or chunk size";
    default: return status > 0 ? "HIP launch error (positive hipError_t)" : "unknown status";
  }
}
