/* C module of the Swift package: the library's C ABI and the HIP runtime
 * calls the Swift side needs to own device buffers and streams. */
#ifndef CRWKVHIP_H
#define CRWKVHIP_H
#include <hip/hip_runtime_api.h>
#include "../../../../include/rwkv_hip.h"
#endif
