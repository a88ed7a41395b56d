// Internal host-side declarations shared by the C-ABI translation units.
#ifndef LEO_HOST_H
#define LEO_HOST_H

#include <stdexcept>
#include <string>

#include "leo_hip.h"

namespace leo {

struct Error : std::runtime_error {
    int32_t code;
    Error(int32_t c, const std::string& m) : std::runtime_error(m), code(c) {}
};

void validate_config(const LeoHostConfig& c);
void splitmix64_stream(uint64_t seed, uint64_t* out, uint64_t count);
void model_initialize(const LeoHostConfig& c, LeoModelView& m);
void model_initialize_synthetic(const LeoHostConfig& c, uint32_t topology, float exponent, uint32_t cap, float sigma,
                                LeoModelView& m);
void model_validate(const LeoHostConfig& c, const LeoModelView& m);
void synthetic_stories(uint64_t seed, uint32_t count, double mean, double stddev, uint32_t min_len, uint32_t max_len,
                       uint8_t* bytes, uint64_t capacity, uint64_t* offsets);

// Records the message for leo_hip_last_error and returns the status code.
int32_t set_error(int32_t code, const std::string& message);

template <class F>
int32_t guarded(F&& f) {
    try {
        f();
        return LEO_OK;
    } catch (const Error& e) {
        return set_error(e.code, e.what());
    } catch (const std::bad_alloc&) {
        return set_error(LEO_ERR_OUT_OF_MEMORY, "host allocation failed");
    } catch (const std::exception& e) {
        return set_error(LEO_ERR_INTERNAL, e.what());
    }
}

}  // namespace leo

#endif
