// Version and status-string entry points of libkrsi_hip.so.
#include "krsi.h"

extern "C" {

int krsi_abi_version(void) { return KRSI_ABI_VERSION; }

const char* krsi_error_string(int status) {
  switch (status) {
    case KRSI_OK:
      return "ok";
    case KRSI_ERR_NULL_POINTER:
      return "krsi: a required pointer is NULL";
    case KRSI_ERR_BAD_SHAPE:
      return "krsi: a size is out of the supported range";
    case KRSI_ERR_MISALIGNED:
      return "krsi: a pointer or leading dimension is not 16-byte aligned";
    case KRSI_ERR_WORKSPACE:
      return "krsi: workspace missing or smaller than the *_workspace_bytes() size";
    case KRSI_ERR_UNSUPPORTED:
      return "krsi: unsupported mode or head dim (D must be a multiple of 8, at most 128)";
    case KRSI_ERR_LAUNCH:
      return "krsi: the HIP runtime rejected a kernel launch";
    case KRSI_ERR_BAD_SCALE:
      return "krsi: scale or eps is not finite";
    case KRSI_ERR_TOO_LARGE:
      return "krsi: the problem needs more scratch than the no-allocation entry point's static "
             "16 MiB buffer (use the entry point that takes a workspace)";
    default:
      return "krsi: unknown status";
  }
}

}  // extern "C"
