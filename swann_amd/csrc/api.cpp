// Host-only parts of the C ABI: error state, options, version, device query.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>

#include "common.h"

namespace swann {

static thread_local char g_err[1024] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

void clear_error() { g_err[0] = '\0'; }

namespace {
struct OptionInfo {
    const char* name;
    int def;
    bool (*valid)(int);
};
bool any_bool(int v) { return v == 0 || v == 1; }
const OptionInfo kOptions[kOptCount] = {
    {"search_block", 0, [](int v) { return v == 0 || v == 64 || v == 256 || v == 1024; }},
    {"prune_simt", 0, any_bool},
    {"prune_f32", 0, any_bool},
    {"sweep_sym", -1, [](int v) { return v >= -1 && v <= 1; }},
    {"sweep_waves", 16, [](int v) { return v == 8 || v == 16; }},
    {"sweep_rowscale", 0, any_bool},
    {"sweep_regstage", 0, any_bool},
    {"sweep_sym_fcap", 0, [](int v) { return v >= 0; }},
    {"sweep_noseed", 0, any_bool},
    {"sweep_order", 1, any_bool},
    {"sweep_repair_max", 4, [](int v) { return v >= 0; }},
};
std::atomic<int> g_opt[kOptCount];
// every option starts at its default when the library loads (after kOptions:
// one translation unit initialises in order of definition)
const bool g_opt_init = [] {
    for (int i = 0; i < kOptCount; ++i) g_opt[i].store(kOptions[i].def);
    return true;
}();

int find_option(const char* name) {
    if (!name) return -1;
    for (int i = 0; i < kOptCount; ++i)
        if (strcmp(kOptions[i].name, name) == 0) return i;
    return -1;
}
}  // namespace

int option(Option o) { return g_opt[o].load(std::memory_order_relaxed); }

}  // namespace swann

extern "C" {

const char* swann_last_error(void) { return swann::g_err; }

const char* swann_version(void) { return "swann_amd 0.1.0 gfx950"; }

int swann_set_option(const char* name, int value) {
    swann::clear_error();
    const int i = swann::find_option(name);
    SWANN_REQUIRE(i >= 0, "unknown option %s", name ? name : "(null)");
    SWANN_REQUIRE(swann::kOptions[i].valid(value), "option %s: %d is not one of its values",
                  name, value);
    swann::g_opt[i].store(value, std::memory_order_relaxed);
    return SWANN_OK;
}

int swann_get_option(const char* name, int* value) {
    swann::clear_error();
    const int i = swann::find_option(name);
    SWANN_REQUIRE(i >= 0, "unknown option %s", name ? name : "(null)");
    SWANN_REQUIRE(value, "get_option: value is NULL");
    *value = swann::g_opt[i].load(std::memory_order_relaxed);
    return SWANN_OK;
}

int swann_reset_options(void) {
    for (int i = 0; i < swann::kOptCount; ++i)
        swann::g_opt[i].store(swann::kOptions[i].def, std::memory_order_relaxed);
    return SWANN_OK;
}

int swann_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n;
}

}  // extern "C"
