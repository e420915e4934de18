// C-ABI status plumbing: thread-local last-error text and the library version.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"
#include "../../include/mosaic_amd.h"

namespace mosaic {

static thread_local char g_last_error[512] = "";
static thread_local uint64_t g_launches = 0;

void note_launch() { ++g_launches; }

void set_last_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

}  // namespace mosaic

extern "C" const char* mosaic_last_error(void) { return mosaic::g_last_error; }

extern "C" uint64_t mosaic_launch_count(void) { return mosaic::g_launches; }

extern "C" int mosaic_version(void) { return MOSAIC_AMD_ABI_VERSION; }
