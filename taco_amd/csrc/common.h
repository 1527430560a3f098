// Shared host-side helpers of libhardshell_hip.so: error state, SHA-256.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>

#include "hardshell_hip.h"

namespace hs {

// Records the failure of the current call (thread-local) and returns its status.
hs_status fail(hs_status st, int code, const std::string &msg);
void clear_error();

// A model-file error (crates/hardshell/src/error.rs): the kind and a message.
struct ModelError {
    hs_model_error kind;
    std::string msg;
};

// SHA-256 (FIPS 180-4).
void sha256(const uint8_t *data, size_t len, uint8_t out[32]);

}  // namespace hs
