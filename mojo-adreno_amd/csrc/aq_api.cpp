// Library-level entry points of the aq C ABI (status text, version). Host code only.
#include "../../include/aq.h"

extern "C" const char* aq_status_string(int status) {
  switch (status) {
    case AQ_OK: return "ok";
    case AQ_ERR_SHAPE: return "bad shape: a size is non-positive or not a multiple the layout requires";
    case AQ_ERR_GROUP: return "bad group size: must be a positive multiple of 8 that divides K";
    case AQ_ERR_ALIGN: return "misaligned pointer: packed weights and activations must be 16-byte aligned";
    case AQ_ERR_LAUNCH: return "HIP kernel launch failed";
    case AQ_ERR_NULL: return "a required pointer is NULL";
    case AQ_ERR_CAPACITY: return "size exceeds the kernel's on-chip staging capacity";
    case AQ_ERR_ARG: return "invalid argument";
    default: return "unknown aq status";
  }
}

extern "C" int aq_version(void) { return 100; }
