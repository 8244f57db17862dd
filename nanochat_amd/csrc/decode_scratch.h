/*
 * The no-allocation decode step's static scratch (decode_scratch.hip): its size and the device address of the
 * current device's copy.
 */
#pragma once

#define NC_DECODE_SCRATCH_BYTES (64ll << 20)

/* The current device's scratch address, taken once per device (aborts on a HIP error). */
void *nc_decode_scratch();
