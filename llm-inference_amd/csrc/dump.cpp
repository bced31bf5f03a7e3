// Activation dumps (include/llm_amd/dump.h; src/dump.cu semantics: one fp32 row per call,
// <dir>/<name>.bin truncated on the first write of a name after dump_open, appended after).
#include <errno.h>
#include <stdio.h>
#include <string.h>
#include <sys/stat.h>

#include <set>
#include <string>
#include <vector>

#include "errors.h"
#include "llm_amd/dump.h"

namespace {
std::string g_dir;              // empty: dumping is off
std::set<std::string> g_seen;   // names written since dump_open

bool write_row(const char *name, const float *row, int n) {
    const std::string path = g_dir + "/" + name + ".bin";
    const bool first = g_seen.insert(name).second;
    FILE *f = fopen(path.c_str(), first ? "wb" : "ab");
    if (!f) return llm_fail("dump: cannot open %s: %s", path.c_str(), strerror(errno));
    const size_t put = fwrite(row, sizeof(float), (size_t)n, f);
    const bool ok = fclose(f) == 0 && put == (size_t)n;
    return ok ? true : llm_fail("dump: cannot write %s", path.c_str());
}

// The dumped tensor is whatever the device holds once all work queued so far has finished.
bool fetch(void *host, const void *dev, size_t bytes) {
    return HIP_OK(hipDeviceSynchronize()) &&
           HIP_OK(hipMemcpy(host, dev, bytes, hipMemcpyDeviceToHost));
}
}  // namespace

extern "C" void dump_open(const char *dir) {
    if (!dir || !*dir) {
        llm_fail("dump: no directory");
        return;
    }
    if (mkdir(dir, 0755) != 0 && errno != EEXIST) {
        llm_fail("dump: cannot create %s: %s", dir, strerror(errno));
        return;
    }
    g_dir = dir;
    g_seen.clear();
}

extern "C" void dump_close(void) {
    g_dir.clear();
    g_seen.clear();
}

extern "C" int dump_enabled(void) { return g_dir.empty() ? 0 : 1; }

extern "C" void dump_bf16(const char *name, const bf16 *d_data, int n) {
    if (g_dir.empty() || n <= 0) return;
    std::vector<uint16_t> bits((size_t)n);
    if (!fetch(bits.data(), d_data, bits.size() * 2)) return;
    std::vector<float> row((size_t)n);
    for (int i = 0; i < n; i++) {
        const uint32_t u = (uint32_t)bits[i] << 16;
        memcpy(&row[i], &u, 4);
    }
    write_row(name, row.data(), n);
}

extern "C" void dump_f32(const char *name, const float *d_data, int n) {
    if (g_dir.empty() || n <= 0) return;
    std::vector<float> row((size_t)n);
    if (fetch(row.data(), d_data, row.size() * 4)) write_row(name, row.data(), n);
}
