// C ABI of the KV path: store construction (MK_KV grammar, pools, window rings, page tables), append, attend, rewind,
// sizes, digest.  Conventions follow the reference's capi.cpp: -1 plus a thread-local message, no exception crosses the
// boundary (guarded, capi.cpp:222-245).  The store is the product's own C++ host runtime; the arithmetic is in the HIP
// kernels (kv_store.hip, kv_attn.hip).
#include "../../include/qwen38_kv.h"
#include "kv_launch.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

using namespace qkv;

namespace {

thread_local std::string g_err;

struct HipError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

#define HCK(x)                                                                                                         \
    do {                                                                                                               \
        const hipError_t e_ = (x);                                                                                     \
        if (e_ != hipSuccess) throw HipError(std::string(#x) + ": " + hipGetErrorString(e_));                         \
    } while (0)

constexpr int SLOTS = 17;
constexpr int ATT_BUCKET_ = 640;
constexpr int ATP_ = 32;

struct Spec {
    int kb[SLOTS], vb[SLOTS], kr[SLOTS], vr[SLOTS];
};

// MK_KV grammar (loader.cu:1329-1365): comma-separated items <side><slot>=<bits>[r], side K, V or * (both), slot a
// number (strtol syntax), empty or * (all slots), bits 4..8, r = stored Walsh-Hadamard rotated; empty items are
// skipped and later items override earlier ones.  The accepted strings and the three messages are the reference's.
struct SpecItem {
    bool side[2]; // applies to K, V
    int slot;     // -1: every slot
    int bits;
    int rot;
};

SpecItem parse_item(const std::string & tok, int n_layers) {
    const size_t eq = tok.find('=');
    const char side = tok[0];
    if (eq == std::string::npos || eq == 0 || (side != 'K' && side != 'V' && side != '*'))
        throw std::runtime_error("MK_KV: bad item " + tok);
    SpecItem it{};
    it.side[0] = side != 'V';
    it.side[1] = side != 'K';
    // the format: one digit 4..8, optionally followed by 'r'
    const char * fmt = tok.c_str() + eq + 1;
    const size_t flen = tok.size() - eq - 1;
    const bool digit_ok = flen >= 1 && fmt[0] >= '4' && fmt[0] <= '8';
    const bool suffix_ok = flen == 1 || (flen == 2 && fmt[1] == 'r');
    if (!digit_ok || !suffix_ok) throw std::runtime_error("MK_KV: expected 4..8 or 4r..8r in " + tok);
    it.bits = fmt[0] - '0';
    it.rot = flen == 2;
    // the slot text between the side letter and '='
    const std::string slot_txt(tok, 1, eq - 1);
    it.slot = -1;
    if (!slot_txt.empty() && slot_txt != "*") {
        char * stop = nullptr;
        const long v = strtol(slot_txt.c_str(), &stop, 10);
        if (*stop != '\0' || v < 0 || v >= n_layers)
            throw std::runtime_error("MK_KV: bad slot in " + tok + " (0.." + std::to_string(n_layers - 1) + " or *)");
        it.slot = (int) v;
    }
    return it;
}

void parse_spec(const char * spec, int n_layers, Spec & s) {
    std::fill(s.kb, s.kb + SLOTS, 8);
    std::fill(s.vb, s.vb + SLOTS, 8);
    std::fill(s.kr, s.kr + SLOTS, 0);
    std::fill(s.vr, s.vr + SLOTS, 0);
    if (!spec) return;
    const char * p = spec;
    for (;;) {
        const char * comma = strchr(p, ',');
        const std::string tok = comma ? std::string(p, comma) : std::string(p);
        if (!tok.empty()) {
            const SpecItem it = parse_item(tok, n_layers);
            const int lo = it.slot < 0 ? 0 : it.slot, hi = it.slot < 0 ? n_layers : it.slot + 1;
            for (int k = lo; k < hi; k++) {
                if (it.side[0]) s.kb[k] = it.bits, s.kr[k] = it.rot;
                if (it.side[1]) s.vb[k] = it.bits, s.vr[k] = it.rot;
            }
        }
        if (!comma) break;
        p = comma + 1;
    }
}

int window_start(int L, int win) {
    if (win <= 0) return 0;
    const int ws = (L + ATT_BUCKET_ - 1) / ATT_BUCKET_ - 1 - (win + ATT_BUCKET_ - 1) / ATT_BUCKET_;
    return ws > 0 ? ws * ATT_BUCKET_ : 0;
}
int ring_rows(int win) { return win > 0 ? ((win + ATT_BUCKET_ - 1) / ATT_BUCKET_ + 1) * ATT_BUCKET_ + ATP_ : 0; }

uint64_t dg_hash(const void * p, size_t nb, uint64_t h = 0xcbf29ce484222325ULL) { // engine.cu:1444-1456
    const unsigned char * b = static_cast<const unsigned char *>(p);
    size_t i = 0;
    for (; i + 8 <= nb; i += 8) {
        uint64_t w;
        memcpy(&w, b + i, 8);
        h = (h ^ w) * 0x100000001b3ULL;
        h ^= h >> 31;
    }
    for (; i < nb; i++) h = (h ^ b[i]) * 0x100000001b3ULL;
    return h;
}

struct Store {
    int dev = 0; // the HIP device the store's memory lives on
    int n_layers = 0, n_seq = 0, ctx = 0, page = 0, n_pages = 0, pt_stride = 0, win = 0, kvrc = 0, win_all = 0;
    Spec spec{};
    StoreLayout S{};
    std::vector<int> ptab;
    int * ptab_dev = nullptr;
    std::vector<int> n, top; // per sequence: committed length, rows written (ring_rewind's kv_top)
    std::vector<void *> allocs;
    size_t ring_bytes = 0;
    // workspace of attend (grown on demand)
    void * part = nullptr;
    size_t part_bytes = 0;
    void * ml = nullptr;
    size_t ml_bytes = 0;
    int max_blocks = 0;
    int occupancy = 0; // decode workgroups per CU: 0 = by launch size, 2 or 3 (launch_attn)
    // 25..48 query rows per kv head: one pass of 8-wave workgroups (1), two batches of 24 rows (0), or by format (2):
    // one pass for q8 K and V, two batches for packed sides, whose dequantization done by both waves of a pair makes
    // the one-pass form the slower one there (preset F at T = 8: 105 vs 94 us per layer; all-q8: 36.7 vs 37.1)
    int wide = 2;
    // RoPE table of the Q/K prep calls: [rope_rows][32] (cos, sin), the caller's or the store's own text table
    const float2 * rope = nullptr;
    int rope_rows = 0;
    void * rope_own = nullptr;
    // mk_kv_profile: a pool of event sets recorded around each call's kernels on the launch stream; a set's elapsed times
    // are read only when the pool wraps around or profiling stops, so timed back-to-back calls never wait on the host
    struct EvSet {
        hipEvent_t e[4] = {}; // kernel start / end: attention (0, 1) and combine (2, 3), or append (0, 1)
        int kind = 0;         // 0 free, 1 attend, 2 append
    };
    static constexpr int NEV = 256;
    int prof = 0;
    double prof_acc[4] = {0, 0, 0, 0}; // calls, attention, combine, append (ms)
    std::vector<EvSet> evs;
    int ev_next = 0;

    void * dalloc(size_t bytes) {
        void * p = nullptr;
        HCK(hipMalloc(&p, std::max<size_t>(bytes, 256)));
        allocs.push_back(p);
        HCK(hipMemset(p, 0, std::max<size_t>(bytes, 256)));
        return p;
    }
    ~Store() {
        for (EvSet & es : evs)
            for (hipEvent_t e : es.e)
                if (e) (void) hipEventDestroy(e);
        for (void * p : allocs) (void) hipFree(p);
        for (void * p : retired) (void) hipFree(p);
        if (part) (void) hipFree(part);
        if (ml) (void) hipFree(ml);
        if (rope_own) (void) hipFree(rope_own);
    }
    // Workspace buffers a larger call has replaced.  They stay allocated until the store is freed: work already
    // enqueued, and any HIP graph captured over an earlier call, still hold their addresses (a graph replays the raw
    // kernel arguments), so freeing them here would let a later replay read and write freed device memory.
    // A buffer that has to grow takes at least 1.5 times its old size, so a context that grows step by step
    // reallocates a logarithmic number of times and the retired buffers together stay below twice the live one.
    std::vector<void *> retired;
    void grow(void *& p, size_t & have, size_t need) {
        if (need <= have) return;
        if (have) need = std::max(need, have + have / 2);
        void * q = nullptr;
        HCK(hipMalloc(&q, need));
        if (p) retired.push_back(p);
        p = q;
        have = need;
    }
    size_t main_row(int seq, int g, int p) const {
        const int lp = p / page;
        return (size_t) (g * n_pages + ptab[(size_t) seq * pt_stride + lp]) * page + (p - lp * page);
    }
};

void prof_read(Store & s, Store::EvSet & es) {
    if (!es.kind) return;
    float ms = 0.f;
    if (es.kind == 1) {
        HCK(hipEventSynchronize(es.e[3]));
        s.prof_acc[0] += 1;
        for (int i = 0; i < 2; i++) {
            HCK(hipEventElapsedTime(&ms, es.e[2 * i], es.e[2 * i + 1]));
            s.prof_acc[1 + i] += ms;
        }
    } else {
        HCK(hipEventSynchronize(es.e[1]));
        HCK(hipEventElapsedTime(&ms, es.e[0], es.e[1]));
        s.prof_acc[3] += ms;
    }
    es.kind = 0;
}

// the event set of the next profiled call (nullptr when profiling is off)
Store::EvSet * prof_set(Store & s, int kind) {
    if (!s.prof) return nullptr;
    Store::EvSet & es = s.evs[(size_t) s.ev_next];
    s.ev_next = (s.ev_next + 1) % Store::NEV;
    prof_read(s, es); // (only when the pool wrapped around)
    es.kind = kind;
    return &es;
}


Store * as_store(void * h) {
    if (!h) throw std::runtime_error("null KV store handle");
    return static_cast<Store *>(h);
}

template <class F> int guarded(F f) {
    try {
        return f();
    } catch (const std::exception & e) {
        g_err = e.what();
        return -1;
    } catch (...) {
        g_err = "unknown exception";
        return -1;
    }
}

void check_seq(const Store & s, int seq) {
    if (seq < 0 || seq >= s.n_seq) throw std::runtime_error("sequence " + std::to_string(seq) + " out of range 0.." + std::to_string(s.n_seq - 1));
}
void check_layers(const Store & s, int layer0, int nl) {
    if (nl < 1 || layer0 < 0 || layer0 + nl > s.n_layers)
        throw std::runtime_error("layers " + std::to_string(layer0) + " .. " + std::to_string(layer0 + nl - 1) + " outside 0.." +
                                 std::to_string(s.n_layers - 1));
}

int rewind_seq(Store & s, int seq, int P) {
    check_seq(s, seq);
    if (P < 0) throw std::runtime_error("negative rewind position");
    if (s.kvrc > 0) { // ring_rewind, ck_pool.cu:285-296
        const int p0 = std::max(0, P - s.kvrc), p1 = std::min(P, s.top[seq] - s.kvrc);
        if (p1 > p0) {
            HCK(launch_ring_refill(s.S, seq, s.n_layers, p0, p1, nullptr));
            HCK(hipDeviceSynchronize());
        }
    }
    s.top[seq] = std::min(s.top[seq], P);
    s.n[seq] = std::min(s.n[seq], P);
    return 0;
}

int digest_seq(Store & s, int seq, unsigned long long * out, int cap) {
    check_seq(s, seq);
    HCK(hipDeviceSynchronize());
    const int nn = s.n[seq], rc = s.kvrc, rlo = rc ? std::max(0, nn - rc) : nn;
    std::vector<unsigned long long> v = {0x4d4b444701ULL, (unsigned long long) nn, 0ULL, (unsigned long long) rc, (unsigned long long) rlo,
                                         (unsigned long long) s.n_layers, (unsigned long long) NKV, 0ULL};
    std::vector<unsigned char> vb;
    std::vector<uint16_t> sb;
    for (int l = 0; l < s.n_layers; l++)
        for (int w = 0; w < 2; w++) {
            const SideLayout & sd = s.S.side[l][w];
            const size_t rb = (size_t) row_bytes(sd.bits);
            for (int g = 0; g < NKV; g++) {
                vb.resize(std::max<size_t>(1, (size_t) nn * rb));
                sb.resize(std::max<size_t>(1, (size_t) nn * 8));
                for (int p = 0; p < nn;) { // page by page: rows of a page are contiguous
                    const int cnt = std::min(nn - p, s.page - p % s.page);
                    const size_t r = s.main_row(seq, g, p);
                    HCK(hipMemcpy(vb.data() + (size_t) p * rb, sd.vals + r * rb, (size_t) cnt * rb, hipMemcpyDeviceToHost));
                    HCK(hipMemcpy(sb.data() + (size_t) p * 8, sd.scs + r * 8, (size_t) cnt * 16, hipMemcpyDeviceToHost));
                    p += cnt;
                }
                for (int p = 0; p < nn; p++) v.push_back(dg_hash(sb.data() + (size_t) p * 8, 16, dg_hash(vb.data() + (size_t) p * rb, rb)));
            }
        }
    for (int l = 0; l < s.n_layers; l++)
        for (int w = 0; w < 2; w++) {
            const SideLayout & sd = s.S.side[l][w];
            for (int g = 0; g < NKV; g++) {
                if (!rc || !sd.ring) {
                    v.insert(v.end(), (size_t) (nn - rlo), 0ULL);
                    continue;
                }
                std::vector<int8_t> rv((size_t) rc * HD);
                std::vector<uint16_t> rs((size_t) rc * 8);
                const size_t base = (size_t) (seq * NKV + g) * rc;
                HCK(hipMemcpy(rv.data(), sd.ring + base * HD, rv.size(), hipMemcpyDeviceToHost));
                HCK(hipMemcpy(rs.data(), sd.rsc + base * 8, rs.size() * 2, hipMemcpyDeviceToHost));
                for (int p = rlo; p < nn; p++) {
                    const size_t r = (size_t) (p % rc);
                    v.push_back(dg_hash(rs.data() + r * 8, 16, dg_hash(rv.data() + r * HD, HD)));
                }
            }
        }
    if (out)
        for (int i = 0; i < std::min((int) v.size(), cap); i++) out[i] = v[(size_t) i];
    return (int) v.size();
}

} // namespace

// the text RoPE table of the Q/K prep: row p, pair i = (cos, sin) of p * base^(-2i/64), base 1e7, computed in double
// and rounded to float (loader.cu:1252-1258, mk_shared.cuh:240)
static void use_default_rope(Store & s) {
    if (!s.rope_own) {
        std::vector<float2> t((size_t) s.ctx * 32);
        for (int p = 0; p < s.ctx; p++)
            for (int i = 0; i < 32; i++) {
                const double th = (double) p * std::pow(10000000.0, -2.0 * i / 64.0);
                t[(size_t) p * 32 + i] = make_float2((float) std::cos(th), (float) std::sin(th));
            }
        HCK(hipMalloc(&s.rope_own, t.size() * sizeof(float2)));
        HCK(hipMemcpy(s.rope_own, t.data(), t.size() * sizeof(float2), hipMemcpyHostToDevice));
    }
    s.rope = static_cast<const float2 *>(s.rope_own);
    s.rope_rows = s.ctx;
}

// The workspace of mk_kv_attend_noalloc: a file-scope device array (each GPU the library runs on holds its own copy
// for the life of the process).  Host code never passes the array's name to a kernel: the name is a host-side stand-in,
// so the device address is looked up once per device (hipGetSymbolAddress, with that device current) and kept.
static constexpr size_t NOALLOC_SCRATCH_BYTES = 64ull << 20;
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

static void * noalloc_scratch(int dev) {
    static std::mutex mu;
    static void * addr[64] = {};
    if (dev < 0 || dev >= 64) throw std::runtime_error("device index out of range for the allocation-free call");
    std::lock_guard<std::mutex> lk(mu);
    if (!addr[dev]) {
        void * p = nullptr;
        HCK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) throw std::runtime_error("hipGetSymbolAddress returned no address for the workspace array");
        addr[dev] = p;
    }
    return addr[dev];
}

extern "C" {

const char * mk_last_error(void) { return g_err.c_str(); }

int mk_kv_window_start(int L, int win) { return window_start(L, win); }
int mk_kv_ring_rows(int win) { return ring_rows(win); }
int mk_kv_cap_T(int n, int T) {
    const int lim = ATT_BUCKET_ * ((n + ATT_BUCKET_) / ATT_BUCKET_) - n;
    return T < lim ? T : lim;
}

int mk_kv_parse_spec(const char * kv_spec, int n_layers, int * out) {
    return guarded([&] {
        if (n_layers < 1 || n_layers > SLOTS) throw std::runtime_error("n_layers must be 1..17");
        Spec s;
        parse_spec(kv_spec, n_layers, s);
        for (int i = 0; i < n_layers; i++) {
            out[i] = s.kb[i];
            out[n_layers + i] = s.vb[i];
            out[2 * n_layers + i] = s.kr[i];
            out[3 * n_layers + i] = s.vr[i];
        }
        return 0;
    });
}

void * mk_kv_new(const char * kv_spec, int win, int win_all, int n_layers, int n_seq, int ctx, int page, int n_pages) {
    Store * s = nullptr;
    try {
        if (n_layers < 1 || n_layers > SLOTS) throw std::runtime_error("n_layers must be 1..17");
        if (n_seq < 1 || n_seq > 64) throw std::runtime_error("n_seq must be 1..64");
        if (ctx < 1) throw std::runtime_error("ctx must be positive");
        if (win < 0) throw std::runtime_error("negative window");
        if (page < 0 || page % ATP_) throw std::runtime_error("page must be a multiple of 32 (0: contiguous)");
        s = new Store();
        HCK(hipGetDevice(&s->dev));
        s->n_layers = n_layers;
        s->n_seq = n_seq;
        s->ctx = ctx;
        parse_spec(kv_spec, n_layers, s->spec);
        const int ctx32 = (ctx + ATP_ - 1) / ATP_ * ATP_;
        s->page = page ? page : ctx32;
        s->pt_stride = (ctx + s->page - 1) / s->page;
        s->n_pages = n_pages > 0 ? n_pages : n_seq * s->pt_stride;
        s->win = win;
        s->win_all = win_all;
        s->kvrc = ring_rows(win);
        s->ptab.assign((size_t) n_seq * s->pt_stride, 0);
        for (int q = 0; q < n_seq; q++)
            for (int i = 0; i < s->pt_stride; i++) s->ptab[(size_t) q * s->pt_stride + i] = (q * s->pt_stride + i) % s->n_pages;
        s->n.assign(n_seq, 0);
        s->top.assign(n_seq, 0);
        s->ptab_dev = static_cast<int *>(s->dalloc(s->ptab.size() * sizeof(int)));
        HCK(hipMemcpy(s->ptab_dev, s->ptab.data(), s->ptab.size() * sizeof(int), hipMemcpyHostToDevice));
        StoreLayout & S = s->S;
        S.ptab = s->ptab_dev;
        S.pt_stride = s->pt_stride;
        S.page = s->page;
        S.n_pages = s->n_pages;
        S.kvrc = s->kvrc;
        S.win = win;
        S.n_seq = n_seq;
        const size_t rows = (size_t) NKV * s->n_pages * s->page;
        for (int l = 0; l < n_layers; l++)
            for (int w = 0; w < 2; w++) {
                SideLayout & sd = S.side[l][w];
                sd.bits = (w ? s->spec.vb : s->spec.kb)[l];
                sd.rot = (w ? s->spec.vr : s->spec.kr)[l];
                sd.vals = static_cast<uint8_t *>(s->dalloc(rows * row_bytes(sd.bits)));
                sd.scs = static_cast<uint16_t *>(s->dalloc(rows * 16));
                if (s->kvrc > 0 && (sd.bits != 8 || win_all)) {
                    const size_t rr = (size_t) n_seq * NKV * s->kvrc;
                    sd.ring = static_cast<int8_t *>(s->dalloc(rr * HD));
                    sd.rsc = static_cast<uint16_t *>(s->dalloc(rr * 16));
                    s->ring_bytes += rr * (HD + 16);
                }
            }
        return s;
    } catch (const std::exception & e) {
        g_err = e.what();
        delete s;
        return nullptr;
    } catch (...) {
        g_err = "unknown exception";
        delete s;
        return nullptr;
    }
}

void mk_free(void * h) { delete static_cast<Store *>(h); }

int mk_kv_set_pages(void * h, int seq, const int * pages, int n) {
    return guarded([&] {
        Store & s = *as_store(h);
        check_seq(s, seq);
        if (n < 0 || n > s.pt_stride) throw std::runtime_error("page table longer than ceil(ctx / page)");
        for (int i = 0; i < n; i++)
            if (pages[i] < 0 || pages[i] >= s.n_pages) throw std::runtime_error("physical page " + std::to_string(pages[i]) + " outside the pool");
        for (int i = 0; i < n; i++) s.ptab[(size_t) seq * s.pt_stride + i] = pages[i];
        HCK(hipMemcpy(s.ptab_dev + (size_t) seq * s.pt_stride, s.ptab.data() + (size_t) seq * s.pt_stride, (size_t) s.pt_stride * sizeof(int),
                      hipMemcpyHostToDevice));
        return 0;
    });
}

static int append_impl(void * h, int seq, int layer0, int n_layers, int pos, int T, const void * k, const void * v, int dtype,
                       const float * knw, void * stream) {
    return guarded([&] {
        Store & s = *as_store(h);
        check_seq(s, seq);
        check_layers(s, layer0, n_layers);
        if (T < 1 || pos < 0 || pos + T > s.ctx) throw std::runtime_error("positions outside 0 .. ctx-1");
        if (dtype != 0 && dtype != 1) throw std::runtime_error("dtype: 0 fp32, 1 fp16");
        if (!k || !v) throw std::runtime_error("null K/V pointer");
        if (knw) {
            if (!s.rope) use_default_rope(s);
            if (pos + T > s.rope_rows) throw std::runtime_error("positions beyond the RoPE table");
        }
        Store::EvSet * es = prof_set(s, 2);
        HCK(launch_append(s.S, seq, layer0, n_layers, pos, T, k, v, dtype, static_cast<hipStream_t>(stream), es ? es->e[0] : nullptr,
                          es ? es->e[1] : nullptr, knw, knw ? s.rope : nullptr));
        s.top[seq] = std::max(s.top[seq], pos + T);
        s.n[seq] = std::max(s.n[seq], pos + T);
        return 0;
    });
}

// qs / gs: row strides (floats) of q and gate; qnw: q-norm weights (the Q prep) or null
// ws (optional): a caller-provided workspace of ws_bytes for the segment partials, used instead of the store's own
// (grown on demand) so that the call allocates nothing
// kin / vin (optional): the fused append of mk_kv_append_attend, [n_seq][T][n_layers][4][256] of dtype kdtype
static int attend_impl(void * h, int layer0, int n_layers, int n_seq, const int * seqs, const int * lens, int T, const float * q,
                       int qs, const float * qnw, const float * gate, int gs, float * out, int8_t * q32a, int8_t * q32b, uint16_t * q32m,
                       void * stream, void * ws = nullptr, size_t ws_bytes = 0, const void * kin = nullptr, const void * vin = nullptr,
                       int kdtype = 0, int prefetch_tiles = 0) {
    return guarded([&] {
        Store & s = *as_store(h);
        const bool prefetch = prefetch_tiles > 0; // mk_kv_prefetch: the launch geometry only, no queries or outputs
        if ((kin != nullptr) != (vin != nullptr)) throw std::runtime_error("null K/V pointer");
        if (kin && kdtype != 0 && kdtype != 1) throw std::runtime_error("dtype: 0 fp32, 1 fp16");
        if ((q32a != nullptr) != (q32b != nullptr) || (q32a != nullptr) != (q32m != nullptr))
            throw std::runtime_error("the q32 outputs come as a set: a, b and meta");
        check_layers(s, layer0, n_layers);
        if (T < 1 || T > MAXT) throw std::runtime_error("T must be 1..8");
        if (n_seq < 1 || n_seq > MAX_SEQ) throw std::runtime_error("1..8 sequences per attend call");
        if (!prefetch && (!q || !out)) throw std::runtime_error("null q/out pointer");
        hipStream_t st = static_cast<hipStream_t>(stream);
        AttnArgs a{};
        a.S = s.S;
        a.T = T;
        a.gate = gate;
        a.qs = qs;
        a.gs = gs;
        a.qnw = qnw;
        a.R = GQA * T;
        a.RP = a.R <= 8 ? 8 : a.R <= 16 ? 16 : 24; // T = 1: one 8-row group; T = 2: 16 rows; T >= 3: 24 rows per wave
        a.wide = 0;                                 // (per launch below: T >= 5, by the knob and the launch's formats)
        a.nseq = n_seq;
        int seg_total = 0;
        for (int i = 0; i < n_seq; i++) {
            check_seq(s, seqs[i]);
            for (int j = 0; j < i; j++)
                if (seqs[j] == seqs[i]) throw std::runtime_error("sequence " + std::to_string(seqs[i]) + " listed twice in one attend call");
            const int L = lens[i];
            if (L < T || L > s.ctx) throw std::runtime_error("context length " + std::to_string(L) + " outside T .. ctx");
            if ((L - T + ATT_BUCKET_) / ATT_BUCKET_ != (L - 1 + ATT_BUCKET_) / ATT_BUCKET_)
                throw std::runtime_error("the T rows straddle a 640-position bucket (cap T with mk_kv_cap_T)");
            // with the fused append the call stores positions L - T .. L - 1 first: no gap after the stored rows
            const int n_after = kin ? std::max(s.n[seqs[i]], L) : s.n[seqs[i]], top_after = kin ? std::max(s.top[seqs[i]], L) : s.top[seqs[i]];
            if (kin && L - T > s.n[seqs[i]])
                throw std::runtime_error("appending from position " + std::to_string(L - T) + " leaves a gap after the " +
                                         std::to_string(s.n[seqs[i]]) + " stored positions of sequence " + std::to_string(seqs[i]));
            if (L > n_after)
                throw std::runtime_error("context length " + std::to_string(L) + " beyond the " + std::to_string(s.n[seqs[i]]) +
                                         " positions stored for sequence " + std::to_string(seqs[i]));
            // the window rows ws .. L-1 are read from the ring, which holds the newest kvrc rows written: rows older
            // than top - kvrc have been overwritten by later appends (rewind first to attend there)
            if (s.ring_bytes && top_after - s.kvrc > window_start(L, s.win))
                throw std::runtime_error("context length " + std::to_string(L) + ": its window rows were overwritten in the ring by " +
                                         "positions up to " + std::to_string(top_after - 1) + " (rewind first)");
            SeqDesc & d = a.sd[i];
            d.seq = seqs[i];
            d.L = L;
            d.ws = window_start(L, s.win);
            d.cs = seg_len(L);
            d.nseg = (L + d.cs - 1) / d.cs;
            d.nseg_m = magic31(d.nseg);
            seg_total += d.nseg;
            // pages pbase, pbase + 1, .. for every logical page the context touches: no table lookups in the kernel
            const int * pt = s.ptab.data() + (size_t) d.seq * s.pt_stride;
            const int npg = (L + s.page - 1) / s.page;
            d.pbase = pt[0];
            for (int k = 1; k < npg && d.pbase >= 0; k++)
                if (pt[k] != pt[0] + k) d.pbase = -1;
        }
        if (qnw) {
            if (!s.rope) use_default_rope(s);
            for (int i = 0; i < n_seq; i++)
                if (lens[i] > s.rope_rows) throw std::runtime_error("positions beyond the RoPE table");
            a.rope = s.rope;
        }
        for (int l = 0; l < s.n_layers; l++) {
            a.krot |= (unsigned) s.spec.kr[l] << l;
            a.vrot |= (unsigned) s.spec.vr[l] << l;
        }
        const size_t max_items = (size_t) n_layers * NKV * seg_total;
        const size_t part_need = (max_items * a.R * HD * sizeof(float) + 255) / 256 * 256, ml_need = max_items * a.R * sizeof(float2);
        float * part_base = nullptr;
        float2 * ml_base = nullptr;
        if (prefetch) {
        } else if (ws) {
            if (part_need + ml_need > ws_bytes)
                throw std::runtime_error("the call needs " + std::to_string(part_need + ml_need) + " bytes of attention workspace, more than the " +
                                         std::to_string(ws_bytes) + " available to an allocation-free call");
            part_base = static_cast<float *>(ws);
            ml_base = reinterpret_cast<float2 *>(static_cast<char *>(ws) + part_need);
        } else {
            s.grow(s.part, s.part_bytes, part_need);
            s.grow(s.ml, s.ml_bytes, ml_need);
            part_base = static_cast<float *>(s.part);
            ml_base = static_cast<float2 *>(s.ml);
        }
        Store::EvSet * es = prefetch ? nullptr : prof_set(s, 1); // (a prefetch is not timed)
        size_t item_base = 0;
        AttnArgs groups[MAX_LAYERS]; // at most one launch per layer (no host allocation on this path)
        size_t ng = 0;
        for (int l = 0; l < n_layers;) { // consecutive layers with the same K/V bits share one launch
            const int kb = s.S.side[layer0 + l][0].bits, vb = s.S.side[layer0 + l][1].bits;
            int e = l + 1;
            while (e < n_layers && s.S.side[layer0 + e][0].bits == kb && s.S.side[layer0 + e][1].bits == vb) e++;
            AttnArgs b = a;
            b.layer0 = layer0 + l;
            b.nl = e - l;
            b.side0[0] = s.S.side[b.layer0][0];
            b.side0[1] = s.S.side[b.layer0][1];
            int item = 0;
            for (int i = 0; i < n_seq; i++) {
                b.sd[i].item0 = item;
                item += b.nl * NKV * b.sd[i].nseg;
            }
            b.n_base = item;
            b.wide = a.R > 24 && s.wide == 1; // (2, the default, runs the two batches: the faster form on every format measured)
            b.n_items = item * (b.wide ? 1 : (a.R + a.RP - 1) / a.RP);
            if (!prefetch) {
                b.q = q + (size_t) l * n_seq * T * NH * qs;
                b.out = out + (size_t) l * n_seq * T * NH * HD;
            }
            if (gate) b.gate = gate + (size_t) l * n_seq * T * NH * gs;
            if (qnw) b.qnw = qnw + (size_t) l * HD;
            if (kin) {
                const size_t esz = kdtype ? 2 : 4;
                b.kin = static_cast<const char *>(kin) + (size_t) l * NKV * HD * esz;
                b.vin = static_cast<const char *>(vin) + (size_t) l * NKV * HD * esz;
                b.kin_nl = n_layers;
                b.kin_f16 = kdtype;
            }
            if (q32a) {
                b.q32a = q32a + (size_t) l * n_seq * T * 192 * 16;
                b.q32b = q32b + (size_t) l * n_seq * T * 192 * 16;
                b.q32m = q32m + (size_t) l * n_seq * T * 192 * 4;
            }
            if (!prefetch) {
                b.part = part_base + item_base * a.R * HD;
                b.ml = ml_base + item_base * a.R;
            }
            item_base += (size_t) item;
            fill_head(b);
            groups[ng++] = b;
            l = e;
        }
        if (prefetch) {
            for (size_t g = 0; g < ng; g++)
                HCK(launch_prefetch(groups[g], s.S.side[groups[g].layer0][0].bits, s.S.side[groups[g].layer0][1].bits, prefetch_tiles, st));
            return 0;
        }
        // profiling: the first launch records the start event, the last the end event (kernel timestamps)
        auto ev = [&](int i, size_t g) { return es && ((i % 2 == 0 && g == 0) || (i % 2 == 1 && g + 1 == ng)) ? es->e[i] : nullptr; };
        for (size_t g = 0; g < ng; g++) {
            const AttnArgs & b = groups[g];
            HCK(launch_attn(b, s.S.side[b.layer0][0].bits, s.S.side[b.layer0][1].bits, s.max_blocks, s.occupancy, st, ev(0, g), ev(1, g)));
        }
        for (size_t g = 0; g < ng; g++) HCK(launch_combine(groups[g], st, ev(2, g), ev(3, g)));
        if (kin)
            for (int i = 0; i < n_seq; i++) {
                s.n[seqs[i]] = std::max(s.n[seqs[i]], lens[i]);
                s.top[seqs[i]] = std::max(s.top[seqs[i]], lens[i]);
            }
        return 0;
    });
}

int mk_kv_append(void * h, int seq, int layer0, int n_layers, int pos, int T, const void * k, const void * v, int dtype, void * stream) {
    return append_impl(h, seq, layer0, n_layers, pos, T, k, v, dtype, nullptr, stream);
}

int mk_kv_append_prep(void * h, int seq, int layer0, int n_layers, int pos, int T, const float * k, const float * v, const float * k_norm,
                      void * stream) {
    if (!k_norm) {
        g_err = "null k_norm pointer";
        return -1;
    }
    return append_impl(h, seq, layer0, n_layers, pos, T, k, v, 0, k_norm, stream);
}

int mk_kv_attend(void * h, int layer0, int n_layers, int n_seq, const int * seqs, const int * lens, int T, const float * q, float * out,
                 void * stream) {
    return attend_impl(h, layer0, n_layers, n_seq, seqs, lens, T, q, HD, nullptr, nullptr, HD, out, nullptr, nullptr, nullptr, stream);
}

int mk_kv_prefetch(void * h, int layer0, int n_layers, int n_seq, const int * seqs, const int * lens, int T, int tiles, void * stream) {
    if (tiles < 1 || tiles > 64) {
        g_err = "tiles must be 1..64";
        return -1;
    }
    return attend_impl(h, layer0, n_layers, n_seq, seqs, lens, T, nullptr, HD, nullptr, nullptr, HD, nullptr, nullptr, nullptr, nullptr, stream,
                       nullptr, 0, nullptr, nullptr, 0, tiles);
}

int mk_kv_append_attend(void * h, int layer0, int n_layers, int n_seq, const int * seqs, const int * lens, int T, const void * k, const void * v,
                        int dtype, const float * q, float * out, void * stream) {
    if (!k || !v) {
        g_err = "null K/V pointer";
        return -1;
    }
    return attend_impl(h, layer0, n_layers, n_seq, seqs, lens, T, q, HD, nullptr, nullptr, HD, out, nullptr, nullptr, nullptr, stream, nullptr, 0,
                       k, v, dtype);
}

int mk_kv_attend_noalloc(void * h, int layer0, int n_layers, int n_seq, const int * seqs, const int * lens, int T, const float * q,
                         float * out, void * stream) {
    void * ws = nullptr;
    const int r = guarded([&] {
        const Store & s = *as_store(h);
        int dev = -1;
        HCK(hipGetDevice(&dev));
        if (dev != s.dev)
            throw std::runtime_error("the current device (" + std::to_string(dev) + ") is not the store's (" + std::to_string(s.dev) + ")");
        ws = noalloc_scratch(dev);
        return 0;
    });
    if (r < 0) return r;
    return attend_impl(h, layer0, n_layers, n_seq, seqs, lens, T, q, HD, nullptr, nullptr, HD, out, nullptr, nullptr, nullptr, stream, ws,
                       NOALLOC_SCRATCH_BYTES);
}

int mk_kv_attend_gated(void * h, int layer0, int n_layers, int n_seq, const int * seqs, const int * lens, int T, const float * q,
                       const float * gate, float * out, void * q32a, void * q32b, unsigned short * q32meta, void * stream) {
    if (!gate) {
        g_err = "null gate pointer";
        return -1;
    }
    return attend_impl(h, layer0, n_layers, n_seq, seqs, lens, T, q, HD, nullptr, gate, HD, out, static_cast<int8_t *>(q32a),
                       static_cast<int8_t *>(q32b), q32meta, stream);
}

int mk_kv_attend_prep(void * h, int layer0, int n_layers, int n_seq, const int * seqs, const int * lens, int T, const float * qg,
                      const float * q_norm, float * out, void * q32a, void * q32b, unsigned short * q32meta, void * stream) {
    if (!qg || !q_norm) {
        g_err = "null qg / q_norm pointer";
        return -1;
    }
    return attend_impl(h, layer0, n_layers, n_seq, seqs, lens, T, qg, 2 * HD, q_norm, qg + HD, 2 * HD, out, static_cast<int8_t *>(q32a),
                       static_cast<int8_t *>(q32b), q32meta, stream);
}

// prefill: the chunk pos .. pos+T-1 in pieces ending at 640-bucket boundaries; each piece's K/V rows are stored, then
// every layer's queries of the piece attend (prefill_host.cu:606-615).  k, v: [T][n_layers][4][256]; q: [n_layers][T][24][qs];
// out: [n_layers][T][24][256]; gate [n_layers][T][24][gs]; q32 [n_layers][T][192][16 | 4].
static int prefill_impl(void * h, int seq, int layer0, int n_layers, int pos, int T, const void * k, const void * v, int dtype,
                        const float * knw, const float * q, int qs, const float * qnw, const float * gate, int gs, float * out,
                        int8_t * q32a, int8_t * q32b, uint16_t * q32m, void * stream) {
    return guarded([&] {
        Store & s = *as_store(h);
        check_seq(s, seq);
        check_layers(s, layer0, n_layers);
        if (T < 1 || pos < 0 || pos + T > s.ctx) throw std::runtime_error("positions outside 0 .. ctx-1");
        if (pos > s.n[seq]) throw std::runtime_error("prefill from position " + std::to_string(pos) + " leaves a gap after the " +
                                                     std::to_string(s.n[seq]) + " stored positions");
        if (dtype != 0 && dtype != 1) throw std::runtime_error("dtype: 0 fp32, 1 fp16");
        if (!k || !v || !q || !out) throw std::runtime_error("null k/v/q/out pointer");
        if ((q32a != nullptr) != (q32b != nullptr) || (q32a != nullptr) != (q32m != nullptr))
            throw std::runtime_error("the q32 outputs come as a set: a, b and meta");
        if (knw || qnw) {
            if (!s.rope) use_default_rope(s);
            if (pos + T > s.rope_rows) throw std::runtime_error("positions beyond the RoPE table");
        }
        hipStream_t st = static_cast<hipStream_t>(stream);
        const size_t esz = dtype ? 2 : 4, krow = (size_t) n_layers * NKV * HD;
        for (int a0 = 0; a0 < T;) {
            const int b = std::min(T, ((pos + a0) / ATT_BUCKET_ + 1) * ATT_BUCKET_ - pos);
            const int n0 = pos + a0, Tp = b - a0;
            HCK(launch_append(s.S, seq, layer0, n_layers, n0, Tp, static_cast<const char *>(k) + a0 * krow * esz,
                              static_cast<const char *>(v) + a0 * krow * esz, dtype, st, nullptr, nullptr, knw, knw ? s.rope : nullptr));
            s.top[seq] = std::max(s.top[seq], n0 + Tp);
            s.n[seq] = std::max(s.n[seq], n0 + Tp);
            PrefillArgs p{};
            p.S = s.S;
            p.seq = seq;
            p.n0 = n0;
            p.Tp = Tp;
            p.L = n0 + Tp;
            p.ws = window_start(p.L, s.win);
            p.R = GQA * Tp;
            p.nrb = (p.R + PF2_ROWS - 1) / PF2_ROWS;
            p.seg = pf_seg(p.L);
            p.nseg = (p.L + p.seg - 1) / p.seg;
            p.qs = qs;
            p.gs = gs;
            p.rope = qnw ? s.rope : nullptr;
            s.grow(s.part, s.part_bytes, (size_t) NKV * p.nseg * p.R * HD * sizeof(float));
            s.grow(s.ml, s.ml_bytes, (size_t) NKV * p.nseg * p.R * sizeof(float2));
            p.part = static_cast<float *>(s.part);
            p.ml = static_cast<float2 *>(s.ml);
            for (int l = 0; l < n_layers; l++) {
                const int sl = layer0 + l;
                const size_t trow = (size_t) l * T + a0; // first token row of the piece in this layer's block
                p.layer = sl;
                p.krot = s.spec.kr[sl];
                p.vrot = s.spec.vr[sl];
                p.q = q + trow * NH * qs;
                p.qnw = qnw ? qnw + (size_t) l * HD : nullptr;
                p.out = out + trow * NH * HD;
                p.gate = gate ? gate + trow * NH * gs : nullptr;
                p.q32a = q32a ? q32a + trow * 192 * 16 : nullptr;
                p.q32b = q32b ? q32b + trow * 192 * 16 : nullptr;
                p.q32m = q32m ? q32m + trow * 192 * 4 : nullptr;
                HCK(launch_prefill(p, s.S.side[sl][0].bits, s.S.side[sl][1].bits, st));
            }
            a0 = b;
        }
        return 0;
    });
}

int mk_kv_prefill(void * h, int seq, int layer0, int n_layers, int pos, int T, const void * k, const void * v, int dtype, const float * q,
                  float * out, void * stream) {
    return prefill_impl(h, seq, layer0, n_layers, pos, T, k, v, dtype, nullptr, q, HD, nullptr, nullptr, HD, out, nullptr, nullptr, nullptr,
                        stream);
}

int mk_kv_prefill_prep(void * h, int seq, int layer0, int n_layers, int pos, int T, const float * k, const float * v, const float * k_norm,
                       const float * qg, const float * q_norm, float * out, void * q32a, void * q32b, unsigned short * q32meta,
                       void * stream) {
    if (!k_norm || !qg || !q_norm) {
        g_err = "null k_norm / qg / q_norm pointer";
        return -1;
    }
    return prefill_impl(h, seq, layer0, n_layers, pos, T, k, v, 0, k_norm, qg, 2 * HD, q_norm, qg + HD, 2 * HD, out,
                        static_cast<int8_t *>(q32a), static_cast<int8_t *>(q32b), q32meta, stream);
}

int mk_kv_set_rope(void * h, const void * table, int rows) {
    return guarded([&] {
        Store & s = *as_store(h);
        if (!table) {
            use_default_rope(s);
            return 0;
        }
        if (rows < 1) throw std::runtime_error("RoPE table rows must be positive");
        s.rope = static_cast<const float2 *>(table);
        s.rope_rows = rows;
        return 0;
    });
}

int mk_kv_rewind(void * h, int seq, int pos) {
    return guarded([&] { return rewind_seq(*as_store(h), seq, pos); });
}
int mk_truncate(void * h, int len) { return mk_kv_rewind(h, 0, len); }
int mk_rewind_to(void * h, int pos) { return mk_kv_rewind(h, 0, pos); }

void mk_kv_sizes(void * h, long long * per_token, long long * rings, long long * state, long long * checkpoint) {
    const Store * s = static_cast<const Store *>(h);
    long long t = 0;
    if (s)
        for (int l = 0; l < s->n_layers; l++)
            for (int w = 0; w < 2; w++) t += (long long) NKV * (row_bytes(s->S.side[l][w].bits) + 16); // host_store.cu:114-120
    if (per_token) *per_token = t;
    if (rings) *rings = s ? (long long) s->ring_bytes : 0;
    if (state) *state = 0;
    if (checkpoint) *checkpoint = 0;
}

int mk_kv_state_digest(void * h, int seq, unsigned long long * out, int cap) {
    return guarded([&] { return digest_seq(*as_store(h), seq, out, cap); });
}
int mk_state_digest(void * h, unsigned long long * out, int cap) { return mk_kv_state_digest(h, 0, out, cap); }

int mk_kv_read_rows(void * h, int seq, int layer, int w, int g, int p0, int n, int ring, void * vals, unsigned short * scales) {
    return guarded([&] {
        Store & s = *as_store(h);
        check_seq(s, seq);
        check_layers(s, layer, 1);
        if (w < 0 || w > 1 || g < 0 || g >= NKV) throw std::runtime_error("side / kv head out of range");
        if (p0 < 0 || n < 0 || p0 + n > s.ctx) throw std::runtime_error("rows outside 0 .. ctx-1");
        const SideLayout & sd = s.S.side[layer][w];
        HCK(hipDeviceSynchronize());
        if (ring) {
            if (!sd.ring) throw std::runtime_error("this side has no window ring");
            for (int i = 0; i < n;) { // runs of consecutive ring rows (a run ends where the ring wraps)
                const int slot = (p0 + i) % s.kvrc, cnt = std::min(n - i, s.kvrc - slot);
                const size_t r = (size_t) (seq * NKV + g) * s.kvrc + slot;
                if (vals)
                    HCK(hipMemcpy(static_cast<uint8_t *>(vals) + (size_t) i * HD, sd.ring + r * HD, (size_t) cnt * HD, hipMemcpyDeviceToHost));
                if (scales) HCK(hipMemcpy(scales + (size_t) i * 8, sd.rsc + r * 8, (size_t) cnt * 16, hipMemcpyDeviceToHost));
                i += cnt;
            }
            return HD;
        }
        const size_t rb = (size_t) row_bytes(sd.bits);
        for (int p = p0; p < p0 + n;) {
            const int cnt = std::min(p0 + n - p, s.page - p % s.page);
            const size_t r = s.main_row(seq, g, p);
            if (vals) HCK(hipMemcpy(static_cast<uint8_t *>(vals) + (size_t) (p - p0) * rb, sd.vals + r * rb, (size_t) cnt * rb, hipMemcpyDeviceToHost));
            if (scales) HCK(hipMemcpy(scales + (size_t) (p - p0) * 8, sd.scs + r * 8, (size_t) cnt * 16, hipMemcpyDeviceToHost));
            p += cnt;
        }
        return (int) rb;
    });
}

int mk_kv_write_rows(void * h, int seq, int layer, int w, int g, int p0, int n, int ring, const void * vals, const unsigned short * scales) {
    return guarded([&] {
        Store & s = *as_store(h);
        check_seq(s, seq);
        check_layers(s, layer, 1);
        if (w < 0 || w > 1 || g < 0 || g >= NKV) throw std::runtime_error("side / kv head out of range");
        if (p0 < 0 || n < 0 || p0 + n > s.ctx) throw std::runtime_error("rows outside 0 .. ctx-1");
        if (!vals || !scales) throw std::runtime_error("null rows / scales");
        const SideLayout & sd = s.S.side[layer][w];
        HCK(hipDeviceSynchronize());
        if (ring) {
            if (!sd.ring) throw std::runtime_error("this side has no window ring");
            if (n > s.kvrc) throw std::runtime_error("more rows than the ring holds");
            for (int i = 0; i < n; i++) {
                const size_t r = (size_t) (seq * NKV + g) * s.kvrc + (p0 + i) % s.kvrc;
                HCK(hipMemcpy(sd.ring + r * HD, static_cast<const uint8_t *>(vals) + (size_t) i * HD, HD, hipMemcpyHostToDevice));
                HCK(hipMemcpy(sd.rsc + r * 8, scales + (size_t) i * 8, 16, hipMemcpyHostToDevice));
            }
        } else {
            const size_t rb = (size_t) row_bytes(sd.bits);
            for (int p = p0; p < p0 + n;) {
                const int cnt = std::min(p0 + n - p, s.page - p % s.page);
                const size_t r = s.main_row(seq, g, p);
                HCK(hipMemcpy(sd.vals + r * rb, static_cast<const uint8_t *>(vals) + (size_t) (p - p0) * rb, (size_t) cnt * rb, hipMemcpyHostToDevice));
                HCK(hipMemcpy(sd.scs + r * 8, scales + (size_t) (p - p0) * 8, (size_t) cnt * 16, hipMemcpyHostToDevice));
                p += cnt;
            }
        }
        s.n[seq] = std::max(s.n[seq], p0 + n);
        s.top[seq] = std::max(s.top[seq], p0 + n);
        return 0;
    });
}

// ring snapshot: header of 8 int64 [magic, version 1, kvrc, ring sides, position, n_layers, 0, 0], then per (slot, side)
// with a ring, in slot order, K before V: the sequence's ring values [NKV][kvrc][256] and scales [NKV][kvrc][8] fp16
static constexpr long long RING_SNAP_MAGIC = 0x4d4b52494e47ll; // "MKRING"
static long long ring_snap_bytes(const Store & s, int & sides) {
    sides = 0;
    for (int l = 0; l < s.n_layers; l++)
        for (int w = 0; w < 2; w++) sides += s.S.side[l][w].ring != nullptr;
    return 64 + (long long) sides * NKV * s.kvrc * (HD + 16);
}

long long mk_kv_ring_snapshot(void * h, int seq, void * dst, long long cap) {
    long long r = -1;
    const int st = guarded([&] {
        Store & s = *as_store(h);
        check_seq(s, seq);
        int sides = 0;
        const long long need = ring_snap_bytes(s, sides);
        r = need;
        if (!dst || cap < need) return 0;
        HCK(hipDeviceSynchronize());
        const long long hdr[8] = {RING_SNAP_MAGIC, 1, s.kvrc, sides, s.n[seq], s.n_layers, 0, 0};
        HCK(hipMemcpy(dst, hdr, sizeof hdr, hipMemcpyDefault));
        uint8_t * o = static_cast<uint8_t *>(dst) + 64;
        const size_t vb = (size_t) NKV * s.kvrc * HD, sb = (size_t) NKV * s.kvrc * 16;
        for (int l = 0; l < s.n_layers; l++)
            for (int w = 0; w < 2; w++) {
                const SideLayout & sd = s.S.side[l][w];
                if (!sd.ring) continue;
                HCK(hipMemcpy(o, sd.ring + (size_t) seq * vb, vb, hipMemcpyDefault));
                HCK(hipMemcpy(o + vb, reinterpret_cast<const uint8_t *>(sd.rsc) + (size_t) seq * sb, sb, hipMemcpyDefault));
                o += vb + sb;
            }
        return 0;
    });
    return st < 0 ? -1 : r;
}

int mk_kv_ring_restore(void * h, int seq, int pos, const void * src, long long bytes) {
    return guarded([&] {
        Store & s = *as_store(h);
        check_seq(s, seq);
        int sides = 0;
        const long long need = ring_snap_bytes(s, sides);
        if (!src || bytes < need) throw std::runtime_error("ring snapshot too small for this store");
        long long hdr[8];
        HCK(hipMemcpy(hdr, src, sizeof hdr, hipMemcpyDefault));
        if (hdr[0] != RING_SNAP_MAGIC || hdr[1] != 1) throw std::runtime_error("not a ring snapshot");
        if (hdr[2] != s.kvrc || hdr[3] != sides || hdr[5] != s.n_layers) throw std::runtime_error("ring snapshot of a different store layout");
        const int snap = (int) hdr[4];
        if (pos < 0 || pos > snap) throw std::runtime_error("restore position beyond the snapshot's position");
        if (pos > s.n[seq]) throw std::runtime_error("restore position beyond the stored rows");
        HCK(hipDeviceSynchronize());
        const uint8_t * in = static_cast<const uint8_t *>(src) + 64;
        const size_t vb = (size_t) NKV * s.kvrc * HD, sb = (size_t) NKV * s.kvrc * 16;
        for (int l = 0; l < s.n_layers; l++)
            for (int w = 0; w < 2; w++) {
                const SideLayout & sd = s.S.side[l][w];
                if (!sd.ring) continue;
                HCK(hipMemcpy(sd.ring + (size_t) seq * vb, in, vb, hipMemcpyDefault));
                HCK(hipMemcpy(reinterpret_cast<uint8_t *>(sd.rsc) + (size_t) seq * sb, in + vb, sb, hipMemcpyDefault));
                in += vb + sb;
            }
        // the window rows the snapshot does not hold (positions before snap - kvrc) come from the main rows, as a rewind
        s.top[seq] = snap;
        return rewind_seq(s, seq, pos);
    });
}

int mk_kv_profile(void * h, int enable, double * out, int cap) {
    return guarded([&] {
        Store & s = *as_store(h);
        if (s.prof)
            for (Store::EvSet & es : s.evs) prof_read(s, es);
        if (enable) {
            if (s.evs.empty()) {
                s.evs.resize(Store::NEV);
                for (Store::EvSet & es : s.evs)
                    for (hipEvent_t & e : es.e) HCK(hipEventCreateWithFlags(&e, hipEventDisableSystemFence));
            }
            for (double & x : s.prof_acc) x = 0;
            s.ev_next = 0;
        }
        const int n = std::min(cap, 4);
        for (int i = 0; i < n; i++) out[i] = s.prof_acc[i];
        s.prof = enable;
        return n;
    });
}

int mk_kv_config(void * h, const char * key, long long value) {
    return guarded([&] {
        Store & s = *as_store(h);
        if (!key) throw std::runtime_error("null key");
        if (!strcmp(key, "max_blocks")) {
            if (value < 0) throw std::runtime_error("max_blocks must be >= 0");
            s.max_blocks = (int) value;
            return 0;
        }
        if (!strcmp(key, "wide")) {
            if (value < 0 || value > 2) throw std::runtime_error("wide must be 0 (two 24-row passes), 1 (one pass) or 2 (by format)");
            s.wide = (int) value;
            return 0;
        }
        if (!strcmp(key, "occupancy")) {
            if (value != 0 && value != 2 && value != 3) throw std::runtime_error("occupancy must be 0 (by launch size), 2 or 3");
            s.occupancy = (int) value;
            return 0;
        }
        throw std::runtime_error(std::string("unknown knob ") + key);
    });
}

} // extern "C"
