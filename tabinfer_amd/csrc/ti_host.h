// ti_host.h — host-side error plumbing shared by every libtabinfer source. No HIP here:
// the host-only parts of the library (the .cpu.bin reader, the error text) also build
// with a plain C++ compiler, which is how the sanitizer tests compile them.
#pragma once
#include <stdint.h>
#include <stddef.h>
#include "../../include/ti.h"

// records the thread's last error message (printf-style) and returns code
int ti_fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

#define TI_CHECK_CTX(ctx) do { if (!(ctx)) return ti_fail(TI_ERR_INVALID, "%s: null context", __func__); } while (0)
#define TI_REQUIRE(cond, ...) do { if (!(cond)) return ti_fail(TI_ERR_INVALID, __VA_ARGS__); } while (0)
