// C entry point over the reference's own Gaussian-noise generator, compiled
// together with the reference source file src/sampler/sampler.cpp (read in
// place from the reference checkout; nothing of it is copied here). Used only
// by tests to pin the oracle's restatement of fill_gaussian_noise bit for bit.
#include "sampler/sampler.h"

extern "C" int ref_fill_gaussian_noise(float* output, unsigned long long count, unsigned int seed,
                                       unsigned long long stream)
{
    return seedvr2::fill_gaussian_noise(output, static_cast<std::size_t>(count), seed, stream) ? 0 : -1;
}
