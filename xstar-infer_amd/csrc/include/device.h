#pragma once

/**
 * Where a Tensor's buffer lives.  The name CUDA is the reference's Python-visible
 * name (xstar_cpp/include/device.h:6-10), kept so callers drop in unchanged; on
 * this build it means HIP device memory on the current MI355X.
 */
enum class Device
{
    CPU,
    CUDA,
};
