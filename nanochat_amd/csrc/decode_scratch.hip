/*
 * The static scratch of nc_decode_step_fp8_noalloc (decode_attn.hip), in a translation unit of its own: compiled
 * without relocatable device code, every .hip file of the library is a code object of its own, and HIP loads a
 * code object on a device only when one of its symbols is first used there. So only a device on which the
 * no-allocation entry runs reserves these bytes (until the process ends); the decode kernels' code object holds
 * none of them.
 *
 * The array's name is a host-side stand-in, never a device address: nc_decode_scratch() takes the device address
 * once per device, with that device current (hipGetSymbolAddress), and callers pass that address to the kernels.
 */
#include <mutex>

#include "common.h"
#include "decode_scratch.h"

#define NC_MAX_DEVICES 64

static __device__ __align__(256) unsigned char scratch[NC_DECODE_SCRATCH_BYTES];

void *nc_decode_scratch() {
    static void *address[NC_MAX_DEVICES];
    static std::mutex lock;
    int dev = 0;
    NC_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= NC_MAX_DEVICES) {
        fprintf(stderr, "decode_scratch.hip: device %d past the %d the scratch table holds\n", dev, NC_MAX_DEVICES);
        abort();
    }
    std::lock_guard<std::mutex> guard(lock);
    if (!address[dev]) {
        void *p = nullptr;
        NC_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        address[dev] = p;
    }
    return address[dev];
}
