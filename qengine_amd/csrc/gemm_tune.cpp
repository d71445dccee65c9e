// GEMM tuning table (see gemm_tune.hpp). File format (text):
//   qengine_amd gemm tune v1 cfg=256x256,256x128 ks=1,2,4
//   device <pci bus id> <cus>          (a section per device)
//   <fmt> <n> <k> <bucket> <glu> <cfg> <ks>
#include "gemm_tune.hpp"

#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <sstream>
#include <string>

namespace {

const char* const kHeader = "qengine_amd gemm tune v1 cfg=256x256,256x128 ks=1,2,4";
std::mutex g_mu;
std::map<std::string, std::map<GemmKey, GemmChoice>> g_tab;  // device line -> choices
std::string g_path;

// the device's line, built once per device index (the PCI bus id and CU count do not change while the process runs):
// every prefill GEMM call looks its choice up, and the HIP queries and string formatting are host cost on each call
constexpr int kMaxDevLines = 64;
std::string g_dev_lines[kMaxDevLines];  // guarded by g_mu

std::string dev_line_uncached(int dev) {
    char bus[64] = "?";
    if (hipDeviceGetPCIBusId(bus, sizeof(bus), dev) != hipSuccess) snprintf(bus, sizeof(bus), "dev%d", dev);
    int cus = 0;
    HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    std::ostringstream o;
    o << "device " << bus << " " << cus;
    return o.str();
}

std::string dev_line() {
    int dev = 0;
    HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevLines) return dev_line_uncached(dev);
    {
        std::lock_guard<std::mutex> lk(g_mu);
        if (!g_dev_lines[dev].empty()) return g_dev_lines[dev];
    }
    const std::string l = dev_line_uncached(dev);
    std::lock_guard<std::mutex> lk(g_mu);
    g_dev_lines[dev] = l;
    return l;
}

void load_locked() {
    FILE* f = fopen(g_path.c_str(), "r");
    if (!f) return;
    char line[512];
    std::map<std::string, std::map<GemmKey, GemmChoice>> tab;
    std::string cur;
    bool ok = fgets(line, sizeof(line), f) && strncmp(line, kHeader, strlen(kHeader)) == 0;
    while (ok && fgets(line, sizeof(line), f)) {
        if (strncmp(line, "device ", 7) == 0) {
            cur = line;
            while (!cur.empty() && (cur.back() == '\n' || cur.back() == '\r')) cur.pop_back();
            continue;
        }
        GemmKey k{};
        GemmChoice c{};
        if (sscanf(line, "%d %d %d %d %d %d %d", &k.fmt, &k.n, &k.k, &k.bucket, &k.glu, &c.cfg, &c.ks) != 7 ||
            cur.empty() || c.cfg < 0 || c.cfg > 1 || (c.ks != 1 && c.ks != 2 && c.ks != 4)) {
            ok = false;
            break;
        }
        tab[cur][k] = c;
    }
    fclose(f);
    if (!ok) {
        fprintf(stderr, "qengine_amd: ignoring the GEMM tuning file %s (other build or malformed)\n", g_path.c_str());
        return;
    }
    for (auto& d : tab)
        for (auto& e : d.second) g_tab[d.first].emplace(e.first, e.second);
}

void save_locked() {
    if (g_path.empty()) return;
    const std::string tmp = g_path + ".tmp";
    FILE* f = fopen(tmp.c_str(), "w");
    if (!f) {
        fprintf(stderr, "qengine_amd: cannot write the GEMM tuning file %s\n", tmp.c_str());
        return;
    }
    fprintf(f, "%s\n", kHeader);
    for (auto& d : g_tab) {
        fprintf(f, "%s\n", d.first.c_str());
        for (auto& e : d.second)
            fprintf(f, "%d %d %d %d %d %d %d\n", e.first.fmt, e.first.n, e.first.k, e.first.bucket, e.first.glu,
                    e.second.cfg, e.second.ks);
    }
    const bool good = fclose(f) == 0;
    if (!good || rename(tmp.c_str(), g_path.c_str()) != 0)
        fprintf(stderr, "qengine_amd: cannot write the GEMM tuning file %s\n", g_path.c_str());
}

}  // namespace

int gemm_bucket(int t) {
    int b = 64;
    while (b < t) b *= 2;
    return b;
}

bool gemm_table_find(const GemmKey& key, GemmChoice& ch) {
    {
        std::lock_guard<std::mutex> lk(g_mu);
        if (g_tab.empty()) return false;  // nothing tuned or loaded: no device lookup at all
    }
    const std::string d = dev_line();
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_tab.find(d);
    if (it == g_tab.end()) return false;
    auto e = it->second.find(key);
    if (e == it->second.end()) return false;
    ch = e->second;
    return true;
}

void gemm_table_add(const GemmKey& key, const GemmChoice& ch) {
    const std::string d = dev_line();
    std::lock_guard<std::mutex> lk(g_mu);
    g_tab[d][key] = ch;
    save_locked();
}

void gemm_table_clear() {
    std::lock_guard<std::mutex> lk(g_mu);
    g_tab.clear();
}

size_t gemm_table_size() {
    std::lock_guard<std::mutex> lk(g_mu);
    size_t n = 0;
    for (auto& d : g_tab) n += d.second.size();
    return n;
}

void gemm_tune_file(const char* path) {
    std::lock_guard<std::mutex> lk(g_mu);
    g_path = path ? path : "";
    if (!g_path.empty()) load_locked();
}
