// Library-level entry points: status strings, ABI version, device capabilities.
#include <string.h>

#include "common.h"

extern "C" const char* omni_codec_error_string(int status) {
  switch (status) {
    case OMNI_OK:
      return "ok";
    case OMNI_ERR_INVALID_ARG:
      return "invalid argument: a shape, stride, pointer or flag outside the contract";
    case OMNI_ERR_UNSUPPORTED:
      return "unsupported: no kernel in this library for the requested shape";
    case OMNI_ERR_LAUNCH:
      return "kernel launch failed";
    case OMNI_ERR_DEVICE:
      return "device query failed";
    default:
      return "unknown status";
  }
}

extern "C" int omni_codec_abi_version(void) { return 11; }

extern "C" int omni_codec_capabilities(int device, char* arch, int arch_capacity,
                                       int64_t* lds_bytes, int64_t* compute_units) {
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return OMNI_ERR_DEVICE;
  if (arch && arch_capacity > 0) {
    strncpy(arch, prop.gcnArchName, (size_t)arch_capacity - 1);
    arch[arch_capacity - 1] = '\0';
  }
  if (lds_bytes) *lds_bytes = (int64_t)prop.sharedMemPerBlock;
  if (compute_units) *compute_units = (int64_t)prop.multiProcessorCount;
  return OMNI_OK;
}
