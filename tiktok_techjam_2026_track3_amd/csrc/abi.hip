// Library-level entry points of libmi355attn.so (version, status strings).
#include "common.h"

extern "C" int mi355_version(void) { return 100; }

extern "C" const char* mi355_status_string(int status) {
  switch (status) {
    case MI355_OK: return "ok";
    case MI355_E_NULL_POINTER: return "required pointer is NULL";
    case MI355_E_BAD_SIZE: return "size out of the supported range";
    case MI355_E_BAD_DTYPE: return "dtype not supported by this entry point";
    case MI355_E_ALIGNMENT: return "pointer, stride or inner size violates 16-byte vector access";
    case MI355_E_HEAD_DIM: return "head_dim not supported";
    case MI355_E_UNSUPPORTED: return "argument combination not supported";
    default: break;
  }
  if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
  return "unknown status";
}
