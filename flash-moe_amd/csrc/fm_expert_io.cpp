// fm_expert_io.cpp -- expert files (packed_experts*/layer_XX.bin, tiered
// manifest) and their movement into HBM.  See include/fm_expert_io.h.
//
// Reference behaviour followed:
//   mode detection            generate.h:1813-1848
//   manifest load/validation  config.h:318-408
//   offset lookup             timing.h:138-148
//   split parallel preads     expert_io.h:150-266, 284-329
// The I/O runs on a small pool of std::thread workers doing pread(2); device
// copies go through pinned (hipHostMalloc) staging buffers, two sets that
// alternate so the reads of one batch overlap the copies of the previous one.
#include <errno.h>
#include <fcntl.h>
#include <stdio.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <condition_variable>
#include <deque>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/fm_expert_io.h"
#include "fm_internal.h"

namespace {

// ------------------------------------------------------------------ JSON --
// Just enough JSON for tiered_manifest.json: objects, arrays, strings,
// numbers (integers kept exact up to 2^64), true/false/null.
struct JVal {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    bool b = false;
    bool is_uint = false;  // number written as a plain non-negative integer
    uint64_t u = 0;
    double d = 0.0;
    std::string s;
    std::vector<JVal> arr;
    std::vector<std::pair<std::string, JVal>> obj;

    const JVal *get(const char *key) const {
        if (kind != OBJ) return nullptr;
        for (auto &kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

struct JParser {
    const char *p, *end;
    std::string err;

    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
    }
    bool fail(const char *m) {
        if (err.empty()) err = m;
        return false;
    }
    bool lit(const char *w) {
        size_t n = strlen(w);
        if ((size_t)(end - p) < n || memcmp(p, w, n)) return fail("bad literal");
        p += n;
        return true;
    }
    bool str(std::string &out) {
        if (p >= end || *p != '"') return fail("expected string");
        p++;
        while (p < end && *p != '"') {
            if (*p == '\\') {
                if (++p >= end) return fail("bad escape");
                switch (*p) {
                case 'n': out += '\n'; break;
                case 't': out += '\t'; break;
                case 'r': out += '\r'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'u':  // keys and values here are ASCII; keep the code point's low byte
                    if (end - p < 5) return fail("bad \\u escape");
                    out += (char)strtol(std::string(p + 1, p + 5).c_str(), nullptr, 16);
                    p += 4;
                    break;
                default: out += *p;
                }
                p++;
            } else {
                out += *p++;
            }
        }
        if (p >= end) return fail("unterminated string");
        p++;
        return true;
    }
    bool num(JVal &v) {
        const char *s = p;
        bool plain = true;
        if (p < end && *p == '-') {
            plain = false;
            p++;
        }
        while (p < end && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '+' ||
                           *p == '-')) {
            if (!(*p >= '0' && *p <= '9')) plain = false;
            p++;
        }
        if (p == s) return fail("expected value");
        std::string t(s, p);
        v.kind = JVal::NUM;
        v.d = strtod(t.c_str(), nullptr);
        if (plain) {
            errno = 0;
            v.u = strtoull(t.c_str(), nullptr, 10);
            v.is_uint = errno == 0;
        }
        return true;
    }
    bool value(JVal &v, int depth) {
        if (depth > 32) return fail("nesting too deep");
        ws();
        if (p >= end) return fail("unexpected end");
        char c = *p;
        if (c == '{') {
            v.kind = JVal::OBJ;
            p++;
            ws();
            if (p < end && *p == '}') {
                p++;
                return true;
            }
            for (;;) {
                ws();
                std::string k;
                if (!str(k)) return false;
                ws();
                if (p >= end || *p != ':') return fail("expected ':'");
                p++;
                v.obj.emplace_back(std::move(k), JVal());
                if (!value(v.obj.back().second, depth + 1)) return false;
                ws();
                if (p < end && *p == ',') {
                    p++;
                    continue;
                }
                if (p < end && *p == '}') {
                    p++;
                    return true;
                }
                return fail("expected ',' or '}'");
            }
        }
        if (c == '[') {
            v.kind = JVal::ARR;
            p++;
            ws();
            if (p < end && *p == ']') {
                p++;
                return true;
            }
            for (;;) {
                v.arr.emplace_back();
                if (!value(v.arr.back(), depth + 1)) return false;
                ws();
                if (p < end && *p == ',') {
                    p++;
                    continue;
                }
                if (p < end && *p == ']') {
                    p++;
                    return true;
                }
                return fail("expected ',' or ']'");
            }
        }
        if (c == '"') {
            v.kind = JVal::STR;
            return str(v.s);
        }
        if (c == 't') {
            v.kind = JVal::BOOL;
            v.b = true;
            return lit("true");
        }
        if (c == 'f') {
            v.kind = JVal::BOOL;
            return lit("false");
        }
        if (c == 'n') {
            v.kind = JVal::NUL;
            return lit("null");
        }
        return num(v);
    }
};

bool read_file(const std::string &path, std::string &out) {
    FILE *f = fopen(path.c_str(), "rb");
    if (!f) return false;
    char buf[1 << 16];
    size_t n;
    while ((n = fread(buf, 1, sizeof buf, f)) > 0) out.append(buf, n);
    bool ok = !ferror(f);
    fclose(f);
    return ok;
}

// Unsigned integer member (manifest counts, offsets, sizes); false if absent
// or not a non-negative integer.
bool juint(const JVal *o, const char *key, uint64_t *out) {
    const JVal *v = o ? o->get(key) : nullptr;
    if (!v || v->kind != JVal::NUM || !v->is_uint) return false;
    *out = v->u;
    return true;
}

// Full pread of [off, off+size) -- loops over short reads; false on error/EOF.
bool pread_full(int fd, char *dst, uint64_t off, uint64_t size) {
    while (size) {
        const size_t want = (size_t)std::min<uint64_t>(size, 1ull << 30);
        ssize_t r = pread(fd, dst, want, (off_t)off);
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) return false;
        dst += r;
        off += (uint64_t)r;
        size -= (uint64_t)r;
    }
    return true;
}

// ------------------------------------------------------------ I/O pool --
// A batch of reads: per-slot outstanding chunk counts and failure flags,
// guarded by the pool mutex.
struct IoBatch {
    std::vector<int> remain;
    std::vector<int> bad;
};

struct IoTask {
    int fd;
    char *dst;
    uint64_t off, size;
    IoBatch *batch;
    int slot;
};

class IoPool {
  public:
    explicit IoPool(int n) {
        for (int i = 0; i < n; i++) th_.emplace_back([this] { run(); });
    }
    ~IoPool() {
        {
            std::lock_guard<std::mutex> g(m_);
            stop_ = true;
        }
        cv_work_.notify_all();
        for (auto &t : th_) t.join();
    }
    void submit(const std::vector<IoTask> &tasks) {
        {
            std::lock_guard<std::mutex> g(m_);
            for (auto &t : tasks) q_.push_back(t);
        }
        cv_work_.notify_all();
    }
    std::mutex &mutex() { return m_; }
    std::condition_variable &done_cv() { return cv_done_; }
    int threads() const { return (int)th_.size(); }

  private:
    void run() {
        for (;;) {
            IoTask t;
            {
                std::unique_lock<std::mutex> l(m_);
                cv_work_.wait(l, [this] { return stop_ || !q_.empty(); });
                if (q_.empty()) return;  // stop requested and nothing left
                t = q_.front();
                q_.pop_front();
            }
            const bool ok = pread_full(t.fd, t.dst, t.off, t.size);
            {
                std::lock_guard<std::mutex> g(m_);
                if (!ok) t.batch->bad[t.slot] = 1;
                t.batch->remain[t.slot]--;
            }
            cv_done_.notify_all();
        }
    }
    std::vector<std::thread> th_;
    std::mutex m_;
    std::condition_variable cv_work_, cv_done_;
    std::deque<IoTask> q_;
    bool stop_ = false;
};

// Page-aligned chunks of one blob (expert_io.h:156-170 active_cache_io_split,
// with Linux 4 KB pages): at most `maxc` chunks of at least 1 MB each.
void split_blob(uint64_t size, int maxc, std::vector<std::pair<uint64_t, uint64_t>> &out) {
    out.clear();
    const uint64_t page = 4096, min_chunk = 1 << 20;
    int c = (int)std::min<uint64_t>((uint64_t)maxc, std::max<uint64_t>(1, size / min_chunk));
    if (size % page) c = 1;
    const uint64_t pages = size / page;
    uint64_t cursor = 0;
    for (int i = 0; i < c; i++) {
        uint64_t np = c == 1 ? 0 : pages / c + ((uint64_t)i < pages % c ? 1 : 0);
        uint64_t len = c == 1 ? size : np * page;
        out.emplace_back(cursor, len);
        cursor += len;
    }
}

struct PinnedSet {
    char *host = nullptr;
    size_t cap = 0;
    hipEvent_t ev = nullptr;
    bool pending = false;  // ev recorded after this set's last copies
};

int pinned_reserve(PinnedSet &s, size_t bytes) {
    if (s.pending) {
        hipError_t e = hipEventSynchronize(s.ev);
        s.pending = false;
        if (e != hipSuccess) return fm_fail(FM_ERR_HIP, "staging: hipEventSynchronize: %s", hipGetErrorString(e));
    }
    if (!s.ev) {
        hipError_t e = hipEventCreateWithFlags(&s.ev, hipEventDisableTiming);
        if (e != hipSuccess) return fm_fail(FM_ERR_HIP, "staging: hipEventCreate: %s", hipGetErrorString(e));
    }
    if (s.cap >= bytes) return FM_OK;
    if (s.host) (void)hipHostFree(s.host);
    s.host = nullptr;
    s.cap = 0;
    hipError_t e = hipHostMalloc((void **)&s.host, bytes, hipHostMallocDefault);
    if (e != hipSuccess) {
        s.host = nullptr;
        return fm_fail(FM_ERR_HIP, "staging: hipHostMalloc(%zu): %s", bytes, hipGetErrorString(e));
    }
    s.cap = bytes;
    return FM_OK;
}

void pinned_release(PinnedSet &s) {
    if (s.pending) (void)hipEventSynchronize(s.ev);
    if (s.host) (void)hipHostFree(s.host);
    if (s.ev) (void)hipEventDestroy(s.ev);
    s = PinnedSet();
}

// Read tasks of one operation, one batch slot per chunk: chunk_expert[c],
// chunk_off[c] (offset inside the blob) and chunk_len[c] say where chunk c
// belongs, so its device copy can start as soon as it is read.  missing[k] = 1
// for experts with nothing to read (layer file unavailable, empty entry).
struct ReadPlan {
    IoBatch b;
    std::vector<int> chunk_expert;
    std::vector<uint64_t> chunk_off, chunk_len, sizes;
    std::vector<int> missing;
};

const char *mode_dir(int mode) {
    return mode == FM_STORE_TIERED ? "packed_experts_tiered" : mode == FM_STORE_2BIT ? "packed_experts_2bit"
                                                                                     : "packed_experts";
}

bool exists(const std::string &p) { return access(p.c_str(), F_OK) == 0; }

}  // namespace

struct fm_expert_store {
    std::string dir;
    int mode = 0;
    uint32_t L = 0, E = 0, H = 0, I = 0, G = 0;
    fm_expert_layout lay4{}, lay2{};
    std::vector<fm_expert_extent> ext;  // [L * E]
    std::vector<int> fd;                // [L], -1 = unavailable
    std::vector<uint64_t> fsize;        // [L]
    uint32_t avail = 0, warnings = 0;
    uint64_t max_blob = 0;
    IoPool *pool = nullptr;
    // per-token staging
    PinnedSet set[2];
    int cur = 0;
    bool inflight = false;
    ReadPlan plan;
    int n = 0;
    std::vector<void *> dst;
    hipStream_t stream = nullptr;
    // whole-layer loads
    PinnedSet lset[2];

    const fm_expert_extent &at(int l, int e) const { return ext[(size_t)l * E + e]; }
};

namespace {

int load_manifest(fm_expert_store *s) {
    const std::string path = s->dir + "/packed_experts_tiered/tiered_manifest.json";
    std::string text;
    if (!read_file(path, text)) return fm_fail(FM_ERR_IO, "tiered manifest %s: cannot read", path.c_str());
    JParser jp{text.data(), text.data() + text.size(), {}};
    JVal root;
    if (!jp.value(root, 0)) return fm_fail(FM_ERR_INVALID, "tiered manifest %s: %s", path.c_str(), jp.err.c_str());
    uint64_t nl = 0, ne = 0, sz4 = 0, sz2 = 0;
    if (!juint(&root, "num_layers", &nl) || !juint(&root, "num_experts", &ne))
        return fm_fail(FM_ERR_INVALID, "tiered manifest: num_layers/num_experts missing");
    if (nl != s->L || ne != s->E)
        return fm_fail(FM_ERR_INVALID, "tiered manifest mismatch: %llux%llu vs config %ux%u", (unsigned long long)nl,
                       (unsigned long long)ne, s->L, s->E);
    if (juint(&root, "expert_size_4bit", &sz4) && sz4 && sz4 != s->lay4.size)
        return fm_fail(FM_ERR_INVALID, "tiered manifest: expert_size_4bit %llu vs config %zu",
                       (unsigned long long)sz4, s->lay4.size);
    if (juint(&root, "expert_size_2bit", &sz2) && sz2 && sz2 != s->lay2.size)
        return fm_fail(FM_ERR_INVALID, "tiered manifest: expert_size_2bit %llu vs config %zu",
                       (unsigned long long)sz2, s->lay2.size);
    const JVal *layers = root.get("layers");
    for (uint32_t l = 0; l < s->L; l++) {
        const JVal *lay = layers ? layers->get(std::to_string(l).c_str()) : nullptr;
        const JVal *ex = lay ? lay->get("experts") : nullptr;
        fm_expert_extent *row = &s->ext[(size_t)l * s->E];
        if (!ex || ex->kind != JVal::ARR) {
            // missing layer: all 4-bit at sequential offsets (config.h:361-369)
            s->warnings++;
            for (uint32_t e = 0; e < s->E; e++) row[e] = {(uint64_t)e * s->lay4.size, s->lay4.size, 4, 0};
            continue;
        }
        for (uint32_t e = 0; e < s->E; e++) {
            if (e >= ex->arr.size()) {  // short list: the entry stays empty (calloc in config.h:352)
                s->warnings++;
                row[e] = {0, 0, 0, 0};
                continue;
            }
            const JVal &je = ex->arr[e];
            uint64_t off = 0, size = 0, bits = 0;
            juint(&je, "offset", &off);
            juint(&je, "size", &size);
            juint(&je, "bits", &bits);
            if (bits != 2 && bits != 4) {  // config.h:375-380: warn, treat as 4-bit
                s->warnings++;
                bits = 4;
            }
            row[e] = {off, size, (int32_t)bits, 0};
        }
    }
    return FM_OK;
}

int check_layer(const fm_expert_store *s, int layer, const char *who) {
    if (!s) return fm_fail(FM_ERR_INVALID, "%s: null store", who);
    if (layer < 0 || (uint32_t)layer >= s->L)
        return fm_fail(FM_ERR_INVALID, "%s: layer %d out of range [0, %u)", who, layer, s->L);
    return FM_OK;
}

// Builds the read tasks of n experts into dst[k] (see ReadPlan).
int plan_reads(fm_expert_store *s, int layer, int n, const int *experts, char *const *dst, ReadPlan &rp,
               std::vector<IoTask> &tasks, const char *who) {
    rp.chunk_expert.clear();
    rp.chunk_off.clear();
    rp.chunk_len.clear();
    rp.sizes.assign(n, 0);
    rp.missing.assign(n, 0);
    tasks.clear();
    std::vector<std::pair<uint64_t, uint64_t>> chunks;
    const int fd = s->fd[layer];
    for (int k = 0; k < n; k++) {
        const int e = experts[k];
        if (e < 0 || (uint32_t)e >= s->E) return fm_fail(FM_ERR_INVALID, "%s: expert %d out of range", who, e);
        const fm_expert_extent &x = s->at(layer, e);
        rp.sizes[k] = x.size;
        if (fd < 0 || x.size == 0) {
            rp.missing[k] = 1;
            continue;
        }
        split_blob(x.size, s->pool->threads(), chunks);
        for (auto &c : chunks) {
            rp.chunk_expert.push_back(k);
            rp.chunk_off.push_back(c.first);
            rp.chunk_len.push_back(c.second);
        }
    }
    const size_t nc = rp.chunk_expert.size();
    rp.b.remain.assign(nc, 1);
    rp.b.bad.assign(nc, 0);
    for (size_t c = 0; c < nc; c++) {
        const int k = rp.chunk_expert[c];
        const fm_expert_extent &x = s->at(layer, experts[k]);
        tasks.push_back({fd, dst[k] + rp.chunk_off[c], x.offset + rp.chunk_off[c], rp.chunk_len[c], &rp.b, (int)c});
    }
    return FM_OK;
}

bool all_done(const IoBatch &b) {
    for (int r : b.remain)
        if (r) return false;
    return true;
}

}  // namespace

extern "C" int fm_expert_store_open(const char *model_dir, int mode, uint32_t num_layers, uint32_t num_experts,
                                    uint32_t hidden, uint32_t inter, uint32_t group_size, int io_threads,
                                    fm_expert_store **out) {
    fm_clear_error();
    FM_REQUIRE(model_dir && out, "fm_expert_store_open: null argument");
    FM_REQUIRE(num_layers > 0 && num_experts > 0, "fm_expert_store_open: empty model (%u layers, %u experts)",
               num_layers, num_experts);
    FM_REQUIRE(mode >= FM_STORE_AUTO && mode <= FM_STORE_TIERED, "fm_expert_store_open: bad mode %d", mode);
    *out = nullptr;
    fm_expert_store *s = new fm_expert_store();
    s->dir = model_dir;
    s->L = num_layers;
    s->E = num_experts;
    s->H = hidden;
    s->I = inter;
    s->G = group_size;
    int rc = fm_expert_layout_compute(hidden, inter, group_size, 4, &s->lay4);
    if (rc == FM_OK) rc = fm_expert_layout_compute(hidden, inter, group_size, 2, &s->lay2);
    if (rc != FM_OK) {
        delete s;
        return rc;
    }
    if (mode == FM_STORE_AUTO) {
        // generate.h:1813-1848: tiered manifest first, then 2-bit only when the 4-bit files are absent
        if (exists(s->dir + "/packed_experts_tiered/tiered_manifest.json"))
            mode = FM_STORE_TIERED;
        else if (exists(s->dir + "/packed_experts_2bit/layer_00.bin") &&
                 !exists(s->dir + "/packed_experts/layer_00.bin"))
            mode = FM_STORE_2BIT;
        else
            mode = FM_STORE_4BIT;
    }
    s->mode = mode;
    s->ext.resize((size_t)s->L * s->E);
    if (mode == FM_STORE_TIERED) {
        rc = load_manifest(s);
        if (rc != FM_OK) {
            delete s;
            return rc;
        }
    } else {
        const fm_expert_layout &ly = mode == FM_STORE_2BIT ? s->lay2 : s->lay4;
        for (uint32_t l = 0; l < s->L; l++)
            for (uint32_t e = 0; e < s->E; e++)
                s->ext[(size_t)l * s->E + e] = {(uint64_t)e * ly.size, ly.size, mode == FM_STORE_2BIT ? 2 : 4, 0};
    }
    s->fd.assign(s->L, -1);
    s->fsize.assign(s->L, 0);
    for (uint32_t l = 0; l < s->L; l++) {
        char name[32];
        snprintf(name, sizeof name, "/layer_%02u.bin", l);
        const std::string path = s->dir + "/" + mode_dir(mode) + name;
        const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
        if (fd < 0) continue;
        struct stat st;
        if (fstat(fd, &st) != 0) {
            close(fd);
            continue;
        }
        // expert reads are random: no readahead (generate.h:1873 F_RDAHEAD 0)
        (void)posix_fadvise(fd, 0, 0, POSIX_FADV_RANDOM);
        s->fd[l] = fd;
        s->fsize[l] = (uint64_t)st.st_size;
        s->avail++;
    }
    for (auto &x : s->ext) s->max_blob = std::max<uint64_t>(s->max_blob, x.size);
    s->pool = new IoPool(io_threads > 0 ? std::min(io_threads, 64) : 8);
    *out = s;
    return FM_OK;
}

extern "C" void fm_expert_store_close(fm_expert_store *s) {
    if (!s) return;
    if (s->inflight) {  // drain the reads of an unfinished staging operation
        std::unique_lock<std::mutex> l(s->pool->mutex());
        s->pool->done_cv().wait(l, [s] { return all_done(s->plan.b); });
    }
    delete s->pool;
    for (int fd : s->fd)
        if (fd >= 0) close(fd);
    for (auto &p : s->set) pinned_release(p);
    for (auto &p : s->lset) pinned_release(p);
    delete s;
}

extern "C" int fm_expert_store_get_info(const fm_expert_store *s, fm_expert_store_info *out) {
    fm_clear_error();
    FM_REQUIRE(s && out, "fm_expert_store_get_info: null argument");
    out->mode = s->mode;
    out->num_layers = s->L;
    out->num_experts = s->E;
    out->layers_available = s->avail;
    out->manifest_warnings = s->warnings;
    out->expert_size_4bit = s->lay4.size;
    out->expert_size_2bit = s->lay2.size;
    return FM_OK;
}

extern "C" int fm_expert_get_extent(const fm_expert_store *s, int layer, int expert, fm_expert_extent *out) {
    fm_clear_error();
    int rc = check_layer(s, layer, "fm_expert_get_extent");
    if (rc) return rc;
    FM_REQUIRE(out, "fm_expert_get_extent: null out");
    FM_REQUIRE(expert >= 0 && (uint32_t)expert < s->E, "fm_expert_get_extent: expert %d out of range [0, %u)",
               expert, s->E);
    *out = s->at(layer, expert);
    return FM_OK;
}

extern "C" int fm_expert_layer_bytes(const fm_expert_store *s, int layer, uint64_t *out) {
    fm_clear_error();
    int rc = check_layer(s, layer, "fm_expert_layer_bytes");
    if (rc) return rc;
    FM_REQUIRE(out, "fm_expert_layer_bytes: null out");
    uint64_t m = 0;
    for (uint32_t e = 0; e < s->E; e++) m = std::max<uint64_t>(m, s->at(layer, e).offset + s->at(layer, e).size);
    *out = m;
    return FM_OK;
}

extern "C" int fm_expert_read(fm_expert_store *s, int layer, int n, const int *experts, void *const *host_dst,
                              int *valid) {
    fm_clear_error();
    int rc = check_layer(s, layer, "fm_expert_read");
    if (rc) return rc;
    FM_REQUIRE(n >= 0 && (n == 0 || (experts && host_dst && valid)), "fm_expert_read: bad arguments");
    FM_REQUIRE(!s->inflight, "fm_expert_read: a staging operation is in flight on this store");
    for (int k = 0; k < n; k++) FM_REQUIRE(host_dst[k], "fm_expert_read: null destination %d", k);
    ReadPlan rp;
    std::vector<IoTask> tasks;
    rc = plan_reads(s, layer, n, experts, (char *const *)host_dst, rp, tasks, "fm_expert_read");
    if (rc) return rc;
    s->pool->submit(tasks);
    {
        std::unique_lock<std::mutex> l(s->pool->mutex());
        s->pool->done_cv().wait(l, [&] { return all_done(rp.b); });
    }
    for (int k = 0; k < n; k++) valid[k] = !rp.missing[k];
    for (size_t c = 0; c < rp.chunk_expert.size(); c++)
        if (rp.b.bad[c]) valid[rp.chunk_expert[c]] = 0;
    int loaded = 0;
    for (int k = 0; k < n; k++) loaded += valid[k];
    return loaded;
}

extern "C" int fm_expert_stage_start(fm_expert_store *s, int layer, int n, const int *experts,
                                     void *const *dev_dst, void *stream) {
    fm_clear_error();
    int rc = check_layer(s, layer, "fm_expert_stage_start");
    if (rc) return rc;
    FM_REQUIRE(!s->inflight, "fm_expert_stage_start: previous staging not waited for");
    FM_REQUIRE(n >= 1 && n <= FM_MAX_K + 1 && experts && dev_dst, "fm_expert_stage_start: bad arguments (n=%d)",
               n);
    for (int k = 0; k < n; k++) FM_REQUIRE(dev_dst[k], "fm_expert_stage_start: null destination %d", k);
    const size_t stride = fm_align_up((size_t)s->max_blob, 4096);
    PinnedSet &ps = s->set[s->cur];
    rc = pinned_reserve(ps, stride * (size_t)n);
    if (rc) return rc;
    std::vector<char *> dst(n);
    for (int k = 0; k < n; k++) dst[k] = ps.host + stride * k;
    std::vector<IoTask> tasks;
    rc = plan_reads(s, layer, n, experts, dst.data(), s->plan, tasks, "fm_expert_stage_start");
    if (rc) return rc;
    s->n = n;
    s->dst.assign(dev_dst, dev_dst + n);
    s->stream = fm_stream(stream);
    s->inflight = true;
    s->pool->submit(tasks);
    return FM_OK;
}

extern "C" int fm_expert_stage_wait(fm_expert_store *s, int *valid) {
    fm_clear_error();
    FM_REQUIRE(s && valid, "fm_expert_stage_wait: null argument");
    FM_REQUIRE(s->inflight, "fm_expert_stage_wait: nothing staged");
    PinnedSet &ps = s->set[s->cur];
    const size_t stride = fm_align_up((size_t)s->max_blob, 4096);
    ReadPlan &rp = s->plan;
    const size_t nc = rp.chunk_expert.size();
    std::vector<char> issued(nc, 0);
    for (int k = 0; k < s->n; k++) valid[k] = !rp.missing[k];
    size_t left = nc;
    int rc = FM_OK;
    while (left) {
        std::vector<size_t> ready;
        {
            std::unique_lock<std::mutex> l(s->pool->mutex());
            s->pool->done_cv().wait(l, [&] {
                for (size_t c = 0; c < nc; c++)
                    if (!issued[c] && rp.b.remain[c] == 0) return true;
                return false;
            });
            for (size_t c = 0; c < nc; c++)
                if (!issued[c] && rp.b.remain[c] == 0) {
                    ready.push_back(c);
                    issued[c] = 1;
                    if (rp.b.bad[c]) valid[rp.chunk_expert[c]] = 0;
                }
        }
        for (size_t c : ready) {  // copies are issued outside the lock, chunk by chunk in completion order
            left--;
            const int k = rp.chunk_expert[c];
            if (rp.b.bad[c] || rc != FM_OK) continue;
            hipError_t e = hipMemcpyAsync((char *)s->dst[k] + rp.chunk_off[c], ps.host + stride * k + rp.chunk_off[c],
                                          rp.chunk_len[c], hipMemcpyHostToDevice, s->stream);
            if (e != hipSuccess)
                rc = fm_fail(FM_ERR_HIP, "fm_expert_stage_wait: hipMemcpyAsync: %s", hipGetErrorString(e));
        }
    }
    int loaded = 0;
    for (int k = 0; k < s->n; k++) loaded += valid[k];
    s->inflight = false;
    hipError_t e = hipEventRecord(ps.ev, s->stream);
    if (e == hipSuccess)
        ps.pending = true;
    else if (rc == FM_OK)
        rc = fm_fail(FM_ERR_HIP, "fm_expert_stage_wait: hipEventRecord: %s", hipGetErrorString(e));
    s->cur ^= 1;
    return rc != FM_OK ? rc : loaded;
}

extern "C" int fm_expert_load_layer(fm_expert_store *s, int layer, void *dev_dst, size_t dev_bytes,
                                    const void **blob_table, uint8_t *bits_table, fm_expert_pool *pool_out,
                                    void *stream) {
    fm_clear_error();
    int rc = check_layer(s, layer, "fm_expert_load_layer");
    if (rc) return rc;
    FM_REQUIRE(dev_dst && blob_table && bits_table && pool_out, "fm_expert_load_layer: null argument");
    FM_REQUIRE(!s->inflight, "fm_expert_load_layer: a staging operation is in flight on this store");
    FM_REQUIRE(((uintptr_t)dev_dst & 255) == 0, "fm_expert_load_layer: dev_dst must be 256-byte aligned");
    uint64_t total = 0;
    fm_expert_layer_bytes(s, layer, &total);
    FM_REQUIRE(dev_bytes >= total, "fm_expert_load_layer: dev_bytes %zu < layer bytes %llu", dev_bytes,
               (unsigned long long)total);
    for (uint32_t e = 0; e < s->E; e++) {
        const fm_expert_extent &x = s->at(layer, e);
        const size_t want = x.bits == 2 ? s->lay2.size : s->lay4.size;
        FM_REQUIRE(x.size == want && (x.bits == 2 || x.bits == 4),
                   "fm_expert_load_layer: layer %d expert %d: size %llu does not match a %d-bit blob (%zu)", layer,
                   e, (unsigned long long)x.size, x.bits, want);
        FM_REQUIRE(x.offset % 256 == 0, "fm_expert_load_layer: layer %d expert %d: offset %llu not 256-aligned",
                   layer, e, (unsigned long long)x.offset);
    }
    const int fd = s->fd[layer];
    if (fd < 0) return fm_fail(FM_ERR_IO, "fm_expert_load_layer: layer %d file unavailable", layer);
    if (s->fsize[layer] < total)
        return fm_fail(FM_ERR_IO, "fm_expert_load_layer: layer %d file holds %llu of %llu bytes", layer,
                       (unsigned long long)s->fsize[layer], (unsigned long long)total);
    hipStream_t st = fm_stream(stream);
    // the whole file streams through two pinned 64 MB sets: the reads of
    // chunk i+1 overlap the device copy of chunk i
    const uint64_t CH = 64ull << 20;
    (void)posix_fadvise(fd, 0, 0, POSIX_FADV_SEQUENTIAL);
    std::vector<std::pair<uint64_t, uint64_t>> parts;
    for (uint64_t pos = 0, i = 0; pos < total && rc == FM_OK; pos += CH, i++) {
        PinnedSet &ps = s->lset[i & 1];
        rc = pinned_reserve(ps, CH);
        if (rc) break;
        const uint64_t len = std::min(CH, total - pos);
        IoBatch b;
        b.remain.assign(1, 0);
        b.bad.assign(1, 0);
        split_blob(len, s->pool->threads(), parts);
        std::vector<IoTask> tasks;
        for (auto &c : parts) tasks.push_back({fd, ps.host + c.first, pos + c.first, c.second, &b, 0});
        b.remain[0] = (int)tasks.size();
        s->pool->submit(tasks);
        {
            std::unique_lock<std::mutex> l(s->pool->mutex());
            s->pool->done_cv().wait(l, [&] { return b.remain[0] == 0; });
        }
        if (b.bad[0]) {
            rc = fm_fail(FM_ERR_IO, "fm_expert_load_layer: layer %d: read failed at %llu", layer,
                         (unsigned long long)pos);
            break;
        }
        hipError_t e = hipMemcpyAsync((char *)dev_dst + pos, ps.host, len, hipMemcpyHostToDevice, st);
        if (e == hipSuccess) e = hipEventRecord(ps.ev, st);
        if (e != hipSuccess) {
            rc = fm_fail(FM_ERR_HIP, "fm_expert_load_layer: copy: %s", hipGetErrorString(e));
            break;
        }
        ps.pending = true;
    }
    (void)posix_fadvise(fd, 0, 0, POSIX_FADV_RANDOM);
    if (rc == FM_OK) {
        std::vector<const void *> ptrs(s->E);
        std::vector<uint8_t> bits(s->E);
        for (uint32_t e = 0; e < s->E; e++) {
            ptrs[e] = (const char *)dev_dst + s->at(layer, e).offset;
            bits[e] = (uint8_t)s->at(layer, e).bits;
        }
        hipError_t e = hipMemcpyAsync(blob_table, ptrs.data(), sizeof(void *) * s->E, hipMemcpyHostToDevice, st);
        if (e == hipSuccess) e = hipMemcpyAsync(bits_table, bits.data(), s->E, hipMemcpyHostToDevice, st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);  // the host tables above go out of scope
        if (e != hipSuccess) rc = fm_fail(FM_ERR_HIP, "fm_expert_load_layer: tables: %s", hipGetErrorString(e));
    } else {
        (void)hipStreamSynchronize(st);
    }
    for (auto &p : s->lset)
        if (p.pending) {
            (void)hipEventSynchronize(p.ev);
            p.pending = false;
        }
    if (rc != FM_OK) return rc;
    *pool_out = fm_expert_pool{(const void *const *)blob_table, bits_table, s->E, s->H, s->I, s->G};
    return FM_OK;
}
