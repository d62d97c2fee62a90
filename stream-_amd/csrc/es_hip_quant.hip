// Host side of libes_hip_quant.so: the C ABI declared in include/es_hip_quant.h.
//
// It validates shapes and pointers, turns a queue of products (the reference engine's jobn/run_jobs,
// src/es_engine.c:144-186) into one launch per weight format with a device-side job table, keeps registered host weights
// resident on the device byte-for-byte, and offers the reference's host-memory prototypes (es_matvec /
// es_matvec_multi, src/es_quant.h:44-47) on top. There is no CPU compute path: without a gfx950 device every compute entry
// point fails with ES_HIP_ENODEV.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <functional>
#include <array>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "es_hip_common.h"
#include "es_hip_host.h"

using esq::MvJob;
using esq::MvLaunch;

namespace {

thread_local std::string g_err;
std::atomic<int> g_order{ES_HIP_ORDER_X86_CONTRACT};

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_fail(hipError_t e, const char *what) {
    return fail(e == hipErrorOutOfMemory ? ES_HIP_ENOMEM : ES_HIP_ERUNTIME, "%s: %s", what, hipGetErrorString(e));
}

// ---- device discovery ---------------------------------------------------------------------------------------------
struct Device {
    int ok = 0;
    int id = -1;
    int cus = 256;   // compute units (the persistent kernels' grids)
    std::string arch, why;
};

Device &device() {
    static Device d;
    static std::once_flag once;
    std::call_once(once, [] {
        int n = 0;
        hipError_t e = hipGetDeviceCount(&n);
        if (e != hipSuccess || n == 0) {
            d.why = std::string("no HIP device: ") + (e != hipSuccess ? hipGetErrorString(e) : "device count is 0");
            return;
        }
        int cur = 0;
        if (hipGetDevice(&cur) != hipSuccess) cur = 0;
        hipDeviceProp_t p;
        if ((e = hipGetDeviceProperties(&p, cur)) != hipSuccess) {
            d.why = std::string("hipGetDeviceProperties: ") + hipGetErrorString(e);
            return;
        }
        d.arch = p.gcnArchName;
        if (d.arch.compare(0, 6, "gfx950") != 0) {
            d.why = "device " + std::to_string(cur) + " is " + d.arch + ", this library is built for gfx950 only";
            return;
        }
        d.id = cur;
        d.cus = p.multiProcessorCount > 0 ? p.multiProcessorCount : 256;
        d.ok = 1;
    });
    return d;
}

int need_device() {
    Device &d = device();
    if (!d.ok) return fail(ES_HIP_ENODEV, "%s", d.why.c_str());
    return ES_HIP_OK;
}

// ---- formats --------------------------------------------------------------------------------------------------------
struct FmtInfo {
    int be, bb, ab, lpb;
};

bool fmt_info(uint32_t t, FmtInfo &f) {
    switch (t) {
    case ES_HIP_Q4_0: f = {32, 18, 36, 1}; return true;
    case ES_HIP_Q5_0: f = {32, 22, 36, 1}; return true;
    case ES_HIP_Q8_0: f = {32, 34, 36, 1}; return true;
    case ES_HIP_Q2_K: f = {256, 84, 292, 4}; return true;
    case ES_HIP_Q3_K: f = {256, 110, 292, 4}; return true;
    case ES_HIP_Q4_K: f = {256, 144, 292, 4}; return true;
    case ES_HIP_Q5_K: f = {256, 176, 292, 4}; return true;
    case ES_HIP_Q6_K: f = {256, 210, 292, 4}; return true;
    }
    return false;
}

// ---- job batches ----------------------------------------------------------------------------------------------------
constexpr size_t LDS_TARGET = 32 * 1024;   // bytes of chain terms per workgroup when the row length allows
constexpr size_t LDS_MAX = 160 * 1024;      // gfx950 LDS per workgroup
constexpr size_t TARGET_WG = 8192;          // workgroups a launch aims for (256 CUs x 8 resident 4-wave groups x 4)
constexpr int MIN_ITERS = 4;                // row passes per workgroup at least (one pipelined load group)
constexpr size_t CHAIN_MAX = 256;           // rows per chain batch at most
constexpr size_t MIN_WG_BLOCKS = 512;       // blocks per workgroup at least: a workgroup's set-up (job lookup, gathered
                                            // activation loads) is a chain of dependent loads that small launches (an
                                            // MoE layer's experts at a few tokens each) would otherwise repeat per 24 rows

struct Group {
    MvLaunch L{};
    std::vector<MvJob> jobs;
};

struct Req {   // one product as the launch planner sees it
    uint32_t type;
    const void *W, *act;
    float *y;
    int32_t *ints, *aux;
    int r0, r1, cols, na;
    size_t astride, ystride;
    const int *arow;   // optional device gather table: activation q is row arow[q] of act
    int act_rows = 0;  // rows of act a gather may index (0: na)
    const void *W2 = nullptr;   // a gated expert product (Q2_K): the up rows; y then holds h's Q8_K blocks (bytes)
    // a column piece of a longer row (decode kernel only): the whole row's bytes, MV_CHAIN_* flags, the lane chains
    size_t row_bytes = 0;
    int chain = 0;
    float *lanes = nullptr;
};

// whole_row: the row length limit applies (a request the entry point does not cut into column pieces)
int check_req(const Req &q, const FmtInfo &f, bool whole_row = true) {
    if (q.cols <= 0 || q.cols % f.be) return fail(ES_HIP_EINVAL, "type %u: cols %d is not a positive multiple of %d", q.type, q.cols, f.be);
    if (q.r0 < 0 || q.r1 < q.r0) return fail(ES_HIP_EINVAL, "bad row range [%d, %d)", q.r0, q.r1);
    if (q.na < 0) return fail(ES_HIP_EINVAL, "negative activation count %d", q.na);
    if (q.r1 == q.r0 || q.na == 0) return ES_HIP_OK;
    if (!q.W || !q.act || !q.y) return fail(ES_HIP_EINVAL, "null W, activation or output pointer");
    if (reinterpret_cast<uintptr_t>(q.W) & 3) return fail(ES_HIP_EINVAL, "W must be 4-byte aligned");
    if (reinterpret_cast<uintptr_t>(q.W2) & 3) return fail(ES_HIP_EINVAL, "W2 must be 4-byte aligned");
    if ((reinterpret_cast<uintptr_t>(q.act) & 3) || (q.astride & 3))
        return fail(ES_HIP_EINVAL, "activation blocks must be 4-byte aligned (pointer and stride)");
    if (reinterpret_cast<uintptr_t>(q.y) & 3) return fail(ES_HIP_EINVAL, "y must be 4-byte aligned");
    const size_t packed = (size_t)(q.cols / f.be) * f.ab;
    if ((q.na > 1 || q.arow) && q.astride < packed) return fail(ES_HIP_EINVAL, "activation stride %zu < %zu bytes of one activation", q.astride, packed);
    if (q.na > 1 && q.ystride < (size_t)q.r1) return fail(ES_HIP_EINVAL, "ystride %zu < r1 %d: outputs of activations overlap", q.ystride, q.r1);
    const int nbk = q.cols / f.be;
    // the decode kernel keeps one row's float terms in LDS (at one activation per pass: 9 floats per block for the
    // 32-element formats, 2 per superblock for the K-quants)
    static_assert((size_t)esq::mv_row_pitch(true, ES_HIP_MAX_COLS_32 / 32, 1) * 4 <= LDS_MAX &&
                  (size_t)esq::mv_row_pitch(false, ES_HIP_MAX_COLS_256 / 256, 1) * 4 <= LDS_MAX,
                  "the header's row limits fit one row's terms");
    const int cmax = f.be == 32 ? ES_HIP_MAX_COLS_32 : ES_HIP_MAX_COLS_256;
    if (whole_row && q.cols > cmax)
        return fail(ES_HIP_EINVAL, "type %u: cols %d above the %d this library handles (ES_HIP_MAX_COLS_*)", q.type, q.cols, cmax);
    (void)nbk;
    return ES_HIP_OK;
}

int pow2_at_least(int v) {
    int p = 1;
    while (p < v) p <<= 1;
    return p;
}

// waves one row is split over in the decode kernel: a power of two covering ceil(nbk / slots)
int segments(int nbk, int slots) {
    int seg = 1;
    while (seg * slots < nbk) seg <<= 1;
    return seg;
}

// Plan the launches: one per (format, workgroup size). The job order inside a launch is kept.
// Q6_K decode at one activation per pass runs faster at three waves per SIMD than at the four its registers allow: its
// launches reserve 41 KB of LDS per 4-wave workgroup, so three share a CU (config 3's head 5.70 -> 5.86 TB/s, Q6_K
// decode at config 2's shapes 5.54 -> 5.74; same-process pairs)
#ifndef ESQ_Q6K_LDS
#define ESQ_Q6K_LDS 41984
#endif
constexpr int PIECES = 16;   // (in a launch key: column pieces of long rows)
int plan_groups(const std::vector<Req> &reqs, std::vector<Group> &out) {
    out.clear();
    std::map<std::pair<uint32_t, int>, std::vector<const Req *>> by_kind;
    size_t total_blocks = 0;
    for (const Req &q : reqs) {
        FmtInfo f;
        if (!fmt_info(q.type, f)) return fail(ES_HIP_EINVAL, "type %u is not computed by this library", q.type);
        int rc = check_req(q, f);
        if (rc) return rc;
        if (q.r1 == q.r0 || q.na == 0) continue;
        // launches by format and workgroup size; column pieces of long rows (whose chains only the 8-wave launches that
        // take several block groups per wave carry) in launches of their own
        const int seg = segments(q.cols / f.be, 64 / f.lpb);
        by_kind[{q.type, q.row_bytes ? 8 | PIECES : seg <= 4 ? 4 : 8}].push_back(&q);
        total_blocks += (size_t)(q.r1 - q.r0) * (q.cols / f.be);
    }
    // workgroups of about total/TARGET_WG blocks each, each wave making at least MIN_ITERS row passes, so one launch keeps
    // every CU busy whether it holds one matrix or a hundred
    const size_t wg_blocks = std::max<size_t>(MIN_WG_BLOCKS, total_blocks / TARGET_WG);
    for (auto &kv : by_kind) {
        FmtInfo f;
        fmt_info(kv.first.first, f);
        const bool w32 = f.be == 32;
        const int slots = 64 / f.lpb;
        const int waves = kv.first.second & ~PIECES;
        Group g;
        int max_na = 1, max_nbk = 1;
        for (const Req *q : kv.second) {
            max_na = std::max(max_na, q->na);
            max_nbk = std::max(max_nbk, q->cols / f.be);
        }
        g.L.seg_loop = segments(max_nbk, slots) > waves || (kv.first.second & PIECES);
        // activations per pass: 3 in one pass of 4 rather than two passes of 2; at most what keeps one row's terms in LDS.
        // Jobs of different counts (an MoE layer's experts) each take their own width in one launch of mixed widths.
        int nt_cap = 4;
        while (nt_cap > 1 && (size_t)esq::mv_row_pitch(w32, max_nbk, nt_cap) * sizeof(float) > LDS_MAX) nt_cap /= 2;
        auto nt_of = [&](int na) { return std::min(nt_cap, na >= 3 ? 4 : std::max(na, 1)); };
        bool mixed = false;
        for (const Req *q : kv.second) mixed = mixed || nt_of(q->na) != nt_of(kv.second[0]->na);
        g.L.type = static_cast<int>(kv.first.first);
        g.L.nt = mixed ? 0 : nt_of(kv.second[0]->na);
        g.L.waves = waves;
        int tile = 0;
        size_t lds = 0;
        for (const Req *q : kv.second) {
            const int nbk = q->cols / f.be, rows = q->r1 - q->r0, nt = nt_of(q->na);
            const int rpi = nbk <= slots ? slots / nbk : 1;
            const int seg = segments(nbk, slots);
            const int rstep = std::max(1, waves / seg) * rpi;   // rows one pass of the workgroup covers
            const size_t per_row = (size_t)esq::mv_row_pitch(w32, nbk, nt) * sizeof(float);
            if (per_row > LDS_MAX) return fail(ES_HIP_EINVAL, "type %u cols %d: a row needs %zu bytes of LDS", q->type, q->cols, per_row);
            int chain_cap = (int)std::min<size_t>(CHAIN_MAX, std::max<size_t>(1, LDS_TARGET / per_row));
            if (chain_cap >= rstep) chain_cap -= chain_cap % rstep;
            int rpw = (int)std::max<size_t>((size_t)MIN_ITERS * rstep, (wg_blocks + nbk - 1) / nbk);
            rpw = std::min(rpw, (rows + rstep - 1) / rstep * rstep);
            rpw = (rpw + rstep - 1) / rstep * rstep;
            const int chain = std::min(chain_cap, rpw);
            rpw = (rpw + chain - 1) / chain * chain;   // whole chain batches per workgroup
            MvJob j{};
            j.W = static_cast<const uint8_t *>(q->W);
            j.act = static_cast<const uint8_t *>(q->act);
            j.y = q->y;
            j.ints = q->ints;
            j.ints_aux = q->aux;
            j.arow = q->arow;
            j.astride = q->astride ? q->astride : (size_t)nbk * f.ab;
            j.ystride = q->ystride;
            j.row_bytes = q->row_bytes ? q->row_bytes : (size_t)nbk * f.bb;
            j.chain = q->chain;
            j.lanes = q->lanes;
            j.r0 = q->r0;
            j.r1 = q->r1;
            j.cols = q->cols;
            j.na = q->na;
            j.tile0 = tile;
            j.rows_per_wg = rpw;
            j.chain_rows = chain;
            j.nt = nt;
            tile += (rows + rpw - 1) / rpw;
            lds = std::max(lds, (size_t)chain * per_row);
            g.jobs.push_back(j);
        }
        // Q6_K at one activation per pass: LDS reserved so that three 4-wave workgroups share a CU (three waves per SIMD)
        if (ESQ_Q6K_LDS && g.L.type == ES_HIP_Q6_K && g.L.nt == 1 && !g.L.seg_loop) lds = std::max<size_t>(lds, ESQ_Q6K_LDS);
        g.L.grid = tile;
        g.L.lds = lds;
        out.push_back(std::move(g));
    }
    return ES_HIP_OK;
}

int launch_single(const Group &g, hipStream_t s, int order = -1) {
    hipError_t e = esq::mv_launch(g.L, nullptr, 1, g.jobs[0], order >= 0 ? order : g_order.load(), s);
    return e == hipSuccess ? ES_HIP_OK : hip_fail(e, "kernel launch");
}

// ---- batches: decode-kernel launches plus, for large Q4_K batches, pre-passes and one matrix-core launch -------------
std::atomic<int> g_mm_min{8};    // activations per Q4_K product from which the prefill kernel is used (<= 0: never)
std::atomic<int> g_mq_min{8};    // activations per K-quant product from which the small-batch kernel is used (<= 0: never)
std::atomic<int> g_mb_min{2};    // activations per Q4_0/Q5_0 product from which the batched kernel is used (<= 0: never)
std::atomic<int> g_mbm_min{2};   // ... and from which that batched kernel is the matrix-core one (<= 0: never)
std::atomic<int> g_mm6_min{16};  // activations per Q6_K product from which its matrix-core kernel is used (<= 0: never)
std::atomic<int> g_mm2_min{2};   // activations per Q2_K product from which its LDS-staged matrix-core kernel is used
std::atomic<int> g_mk_min{32};   // activations per Q4_K product from which the direct-activation matrix-core kernel is used
std::atomic<int> g_mk_min_tiles{128};   // ... and its 64 x 128 tiles per product from which it is (twice that for K > 4096)
std::atomic<int> g_mk5_min{8};          // activations per Q5_K product from which the direct-activation kernel is used
std::atomic<int> g_mk3_min{8};          // ... per Q3_K product
std::atomic<int> g_mx_max{64};          // activations per Q2_K product up to which the expert-sized kernel is used (2+)
std::atomic<int> g_moe_gated{1};        // MoE layers with Q2_K gate/up and a K-quant down: the gated expert kernel
std::atomic<int> g_mbx_on{1};           // batched 32-wide products on the kernel reading Q8_0 rows (0: the pre-pass one)

struct Prep {   // one activation pre-pass (shared by products that read the same activations)
    const uint8_t *act;
    const int *arow;
    uint64_t astride;
    int na, na_pad, nbk, kind;
    size_t xq_off, xm_off;
};

struct MbGroup {   // one batched 32-wide launch: products of one format on one of the two kernels
    int type;
    bool mfma;
    int grid = 0;
    std::vector<esq::MbJob> jobs;
    size_t off = 0;
};

struct MqGroup {   // one small-batch matrix-core launch: products of one format and activation-tile count
    int type, wn, grid = 0;
    std::vector<esq::MqJob> jobs;
    size_t off = 0;
};

struct MmGroup {   // one matrix-core launch: products of one format sharing a workgroup tile shape
    int type, bm, bn, nw, grid = 0;
    std::vector<esq::MmJob> jobs;
    size_t off = 0;   // byte offset of the job table in the device image
};

struct MkGroup {   // one direct-activation matrix-core launch: products of one format, gathered activations or not
    int type;
    bool gather;
    int nbkm = 0;     // > 0: the expert-sized kernel (es_hip_mx.hip) in LDS size class nbkm
    bool b32 = false; // ... or with nbkm, the 32-wide kernel reading Q8_0 rows (es_hip_mbx.hip)
    int tok = esq::MK_TOK;   // the direct kernel's activations per tile
    bool gated = false;      // with nbkm: the gated expert kernel (gate and up of a Q2_K expert, h as Q8_K blocks)
    int grid = 0;
    std::vector<esq::MkJob> jobs;
    size_t off = 0;
};

// One launch of the persistent direct kernel (es_hip_mk.hip): every eligible product of one format, cut into tiles of
// MK_ROWS rows x 128 or 64 activations and scheduled over the workgroups by the host (pk_schedule).
struct PkGroup {
    int type;
    struct Prod {
        const uint8_t *W, *act;
        float *y;
        uint32_t astride, ystride, row_bytes;
        int r0, r1, nbk, na;
    };
    std::vector<Prod> prods;
    std::vector<esq::PkTile> tiles;   // in workgroup order
    std::vector<int> wgptr;           // grid + 1 entries: workgroup g takes tiles[wgptr[g] .. wgptr[g + 1])
    int grid = 0, g64 = 0;            // workgroups [0, g64) take the 64-wide tiles
    bool ws = false;                  // the wave-specialised form (Q4_K): one workgroup per CU, 128-wide tiles only
    size_t off = 0;                   // byte offset of the tiles in the device image; wgptr follows them
};

struct Batch {
    std::vector<Group> mv;
    std::vector<MkGroup> mkg;
    std::vector<PkGroup> pkg;
    std::vector<Prep> preps;
    std::vector<std::pair<int, esq::MmJob>> mm;   // (type, job); xq / xm hold workspace offsets until bind(); copied into mmg
    std::vector<MmGroup> mmg;
    std::vector<MqGroup> mqg;
    std::vector<MbGroup> mbg;
    std::vector<esq::PrepJob> pj;   // the pre-passes as launched (filled by bind)
    long prep_total = 0;
    size_t prep_off = 0;
    size_t ws_bytes = 0;
    std::vector<size_t> mv_off;   // byte offsets of the job tables in the device image
    size_t table_bytes = 0;
};

std::atomic<int> g_mm_tile{0};   // forced tile for batches of >= 128 activations: bm | bn << 10 | waves << 20 (0: automatic)

// Workgroup tile of a product: the largest (best operand reuse) that still gives every CU a workgroup.
void mm_tile(int type, const esq::MmJob &j, int &bm, int &bn, int &nw) {
    nw = 8;
    if (type == ES_HIP_Q6_K || type == ES_HIP_Q2_K) {   // 128 rows x up to 64 activations (Q2_K: at least 32)
        bm = 128;
        bn = std::min(j.na_pad, 64);
        return;
    }
    if (j.na_pad < 128) {   // small batches: 128 rows x all the activations (16, 32 or 64)
        bm = 128;
        bn = j.na_pad;
        return;
    }
    if (const int f = g_mm_tile.load()) {
        bm = f & 1023;
        bn = (f >> 10) & 1023;
        nw = f >> 20;
        return;
    }
    const int rows = j.r1 - j.r0;
    bm = bn = 128;
    if ((long)((rows + 127) / 128) * (j.na_pad / 128) >= 256) return;
    bm = bn = 64;   // 64 x 64: four times the workgroups
}

size_t align256(size_t v) { return (v + 255) / 256 * 256; }

bool mm_eligible(const Req &q) {
    const int mn = q.type == ES_HIP_Q6_K ? g_mm6_min.load() : q.type == ES_HIP_Q2_K ? g_mm2_min.load() : g_mm_min.load();
    // the Q2_K kernel addresses its weights with 32-bit offsets from row 0 of the matrix
    if (q.type == ES_HIP_Q2_K && (size_t)q.r1 * (size_t)(q.cols / 256) * 84 + 64 >= ((size_t)1 << 32)) return false;
    return (q.type == ES_HIP_Q4_K || q.type == ES_HIP_Q6_K || q.type == ES_HIP_Q2_K) && mn > 0 && q.na >= mn && !q.ints &&
           q.r1 > q.r0;
}

// the direct-activation kernel: Q4_K batches of at least g_mk_min (Q5_K, Q3_K: of at least g_mk5_min, g_mk3_min), every
// activation row
// within 4 GiB of act
// the output stride the direct kernel uses: any stride >= r1 serves a single activation (only its row 0 is written)
size_t mk_ystride(const Req &q) { return q.na > 1 ? q.ystride : std::max(q.ystride, (size_t)q.r1); }

// the expert-sized kernel: Q2_K products of 2 .. g_mx_max activations, rows of at most MX_NBK superblocks, every
// activation row within 4 GiB of act
bool mx_eligible(const Req &q) {
    const int mx = g_mx_max.load();
    if (q.type != ES_HIP_Q2_K || q.na < 2 || q.na > mx || q.ints || q.r1 <= q.r0 || q.cols / 256 > esq::MX_NBK) return false;
    if (q.W2 && (q.r0 % 256 || q.r1 % 256)) return false;   // the gated kernel's tiles are whole blocks of h
    const size_t rows = q.arow ? (size_t)std::max(q.act_rows, 0) : (size_t)q.na;
    const size_t stride = q.astride ? q.astride : (size_t)(q.cols / 256) * 292;
    return (!q.arow || q.act_rows > 0) && rows * stride < ((size_t)1 << 32) - 65536 &&
           ((size_t)q.na + esq::MX_TOK) * mk_ystride(q) * sizeof(float) < ((size_t)1 << 31);
}

std::atomic<int> g_mk_tok64{1};   // the direct kernel's 64-activation tiles for products short of row tiles (0: never)

// the direct kernel's activations per tile: 64 for Q5_K and Q3_K products when 128 would leave fewer than 256 tiles (a
// quarter of the device's workgroup slots) and the batch fills at least one 64-wide tile, else MK_TOK. Q4_K's short
// products keep the LDS-staged kernel instead: config 2's down product at T = 512 took longer on 64-wide direct tiles
// (the prefill step 90.6 -> 97.2 us) while Q5_K's step, which has no other matrix-core kernel, went 128 -> 119 us.
int mk_tok(const Req &q) {
    if (q.type == ES_HIP_Q4_K || !g_mk_tok64.load() || q.na < 64) return esq::MK_TOK;
    const size_t rt = (size_t)((q.r1 - q.r0 + esq::MK_ROWS - 1) / esq::MK_ROWS);
    return rt * ((q.na + esq::MK_TOK - 1) / esq::MK_TOK) < 256 ? 64 : esq::MK_TOK;
}

bool mk_eligible(const Req &q) {
    const bool q5 = q.type == ES_HIP_Q5_K, q3 = q.type == ES_HIP_Q3_K;
    const int mn = q5 ? g_mk5_min.load() : q3 ? g_mk3_min.load() : g_mk_min.load();
    if ((q.type != ES_HIP_Q4_K && !q5 && !q3) || mn <= 0 || q.na < mn || q.ints || q.r1 <= q.r0) return false;
    const size_t rows = q.arow ? (size_t)std::max(q.act_rows, 0) : (size_t)q.na;
    const size_t stride = q.astride ? q.astride : (size_t)(q.cols / 256) * 292;
    // Tiles (64 rows x 128 activations, one workgroup each) against the K loop each runs: measured on config 2's shapes,
    // this kernel wins from 128 tiles of 8 superblocks (8192 x 2048 at 128 activations: 17 us against 28 us) and loses
    // with 128 tiles of 32 superblocks (2048 x 8192 at 512: 60 us against 45 us, a quarter of the chip's workgroup slots
    // each running a long chain); from 256 tiles it wins or ties at every depth. Products short of row tiles take tiles
    // of 64 activations (mk_tok), counted here as they run.
    // Q5_K and Q3_K have no other matrix-core kernel: against the decode kernel's passes of 4 activations it wins at any
    // tile count.
    const int mt = g_mk_min_tiles.load(), tok = mk_tok(q);
    const size_t tiles = (size_t)((q.r1 - q.r0 + esq::MK_ROWS - 1) / esq::MK_ROWS) * ((q.na + tok - 1) / tok);
    if (!q5 && !q3 && (tiles < (size_t)mt || (tiles < 2 * (size_t)mt && q.cols > 16 * 256))) return false;
    // 32-bit offsets: activation rows within 4 GiB of the activation pointer; outputs (with a tile of activations past
    // the last) below 2^31 bytes, the range the kernel's buffer stores are checked against
    return (!q.arow || q.act_rows > 0) && rows * stride < ((size_t)1 << 32) - 65536 &&
           ((size_t)q.na + esq::MK_TOK) * mk_ystride(q) * sizeof(float) < ((size_t)1 << 31);
}

// the persistent direct kernel: 0 off (products take the per-tile launches), 1 automatic (Q4_K launches of at least 4
// tiles of 64 rows x 128 activations per CU take the wave-specialised form, others the two-workgroup form), 2 the
// wave-specialised form for every Q4_K launch, 3 the two-workgroup form for every launch
std::atomic<int> g_pk_on{1};
std::atomic<uint64_t> g_cfg_gen{0};   // bumped by every setting that changes how a batch is planned

// The persistent direct kernel: Q4_K / Q3_K products that the direct kernels take (at least g_mk_min / g_mk3_min
// activations), with an even number (>= 2) of superblocks per row and no gathered activations, every activation row
// within 4 GiB of act and a tile's outputs (128 activations) within 2^31 bytes of its first.
bool pk_eligible(const Req &q) {
    if (!g_pk_on.load() || q.arow || q.ints || q.r1 <= q.r0) return false;
    if (q.type != ES_HIP_Q4_K && q.type != ES_HIP_Q3_K) return false;
    const int mn = q.type == ES_HIP_Q3_K ? g_mk3_min.load() : g_mk_min.load(), nbk = q.cols / 256;
    if (mn <= 0 || q.na < mn || nbk < 2 || (nbk & 1)) return false;
    const size_t stride = q.astride ? q.astride : (size_t)nbk * 292;
    // (a tile's stores past its activations fall outside its range only when consecutive activations' outputs are at
    // least a tile's rows apart)
    return (size_t)q.na * stride < ((size_t)1 << 32) - 65536 && mk_ystride(q) >= (size_t)std::min(esq::MK_ROWS, q.r1 - q.r0) &&
           (size_t)esq::MK_TOK * mk_ystride(q) * sizeof(float) < ((size_t)1 << 31);
}

// Relative cost of a tile: its superblocks (a 64-wide one does ~0.6 of a 128-wide one's work: the same unpacking and
// weight loads for half the matrix work) and a fixed part for its first loads and its stores.
double pk_cost(int nbk, bool t64) { return nbk * (t64 ? 0.6 : 1.0) + 1.0; }

// The schedule of a persistent launch: grid = 2 workgroups per CU; workgroups [0, g64) take 64-wide tiles, the rest
// 128-wide ones. A product takes 64-wide tiles when it has at most 64 activations or when one 128-wide tile would cost
// more than a workgroup's mean load (a long row against few row tiles: config 2's down product). Some 128-wide tiles are
// then cut in two and moved to the 64-wide workgroups until both sets of workgroups carry about the same load. Within
// each set, all tiles of a row tile go to one XCD (workgroup g runs on XCD g % 8: its L2 reads the row tile's weights
// once), row tiles are spread over the XCDs and tiles over an XCD's workgroups longest first, each to the least loaded.
// Returns false when some workgroup would get more than PK_MAX_TILES tiles.
// The form of a persistent launch: the wave-specialised kernel (one workgroup per CU, 128-wide tiles) measured faster
// on config 2's three products in one launch (1152 tiles: 75-77 us against 85-86 us), even with gate and up alone (1024
// tiles), and slower when the tiles leave CUs idle (the down product alone, 128 tiles: 47 us against 37 us).
bool pk_ws(const PkGroup &g, int cus) {
    const int on = g_pk_on.load();
    if (g.type != ES_HIP_Q4_K || on == 3) return false;
    if (on == 2) return true;
    long tiles = 0;
    for (const PkGroup::Prod &p : g.prods)
        tiles += (long)((p.r1 - p.r0 + esq::MK_ROWS - 1) / esq::MK_ROWS) * ((p.na + 127) / 128);
    return tiles >= 4L * std::max(cus, 8);
}

bool pk_schedule_form(PkGroup &g, int cus);

// Schedules a persistent launch in the form pk_ws picks; a wave-specialised schedule with too many tiles for some
// workgroup falls back to the two-workgroup form (twice the workgroups).
bool pk_schedule(PkGroup &g, int cus) {
    g.ws = pk_ws(g, cus);
    if (pk_schedule_form(g, cus)) return true;
    if (!g.ws) return false;
    g.ws = false;
    return pk_schedule_form(g, cus);
}

bool pk_schedule_form(PkGroup &g, int cus) {
    const int G = (g.ws ? 1 : 2) * std::max(cus, 8) / 8 * 8;
    struct Tl { int p, rt, t0, nt; bool t64; double c; };
    std::vector<Tl> v128, v64;
    double mean = 0;
    for (const PkGroup::Prod &p : g.prods)
        mean += (double)((p.r1 - p.r0 + esq::MK_ROWS - 1) / esq::MK_ROWS) * ((p.na + 127) / 128) * pk_cost(p.nbk, false);
    mean /= G;
    for (int pi = 0; pi < (int)g.prods.size(); pi++) {
        const PkGroup::Prod &p = g.prods[pi];
        const int rts = (p.r1 - p.r0 + esq::MK_ROWS - 1) / esq::MK_ROWS;
        const bool t64 = !g.ws && (p.na <= 64 || pk_cost(p.nbk, false) > mean);
        const int T = t64 ? 64 : 128;
        for (int rt = 0; rt < rts; rt++)
            for (int t0 = 0; t0 < p.na; t0 += T)
                (t64 ? v64 : v128).push_back(Tl{pi, rt, t0, std::min(T, p.na - t0), t64, pk_cost(p.nbk, t64)});
    }
    // LPT of a tile set over workgroups [base, base + n) (n a multiple of 8), row tiles kept on one XCD. Row tiles are
    // numbered through rtb (product p's row tile rt is rtb[p] + rt); tiles go longest first (ties in list order), each to
    // the least loaded workgroup of its XCD (ties to the lowest index), through one min-heap per XCD.
    std::vector<int> rtb(g.prods.size() + 1, 0);
    for (size_t pi = 0; pi < g.prods.size(); pi++)
        rtb[pi + 1] = rtb[pi] + (g.prods[pi].r1 - g.prods[pi].r0 + esq::MK_ROWS - 1) / esq::MK_ROWS;
    // seq receives the tiles' indices in the order they were placed and wg_of[i] tile i's workgroup
    auto lpt = [&](const std::vector<Tl> &ts, int base, int n, std::vector<int> &seq, std::vector<int> &wg_of,
                   std::vector<double> &load) {
        std::vector<double> rtc(rtb.back(), 0.0);
        for (const Tl &t : ts) rtc[rtb[t.p] + t.rt] += t.c;
        std::vector<int> order;
        for (int i = 0; i < rtb.back(); i++)
            if (rtc[i] > 0) order.push_back(i);
        std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return rtc[a] > rtc[b]; });
        double xl[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        std::vector<int8_t> xcd(rtb.back(), 0);
        for (int o : order) {
            int x = 0;
            for (int i = 1; i < 8; i++)
                if (xl[i] < xl[x]) x = i;
            xcd[o] = (int8_t)x;
            xl[x] += rtc[o];
        }
        seq.resize(ts.size());
        for (size_t i = 0; i < ts.size(); i++) seq[i] = (int)i;
        std::stable_sort(seq.begin(), seq.end(), [&](int a, int b) { return ts[a].c > ts[b].c; });
        wg_of.assign(ts.size(), -1);
        typedef std::pair<double, int> LW;   // (load, workgroup)
        std::vector<LW> heap[8];
        for (int w = base; w < base + n; w++) heap[w % 8].push_back({load[w], w});
        for (auto &h : heap) std::make_heap(h.begin(), h.end(), std::greater<LW>());
        for (int i : seq) {
            std::vector<LW> &h = heap[xcd[rtb[ts[i].p] + ts[i].rt]];
            std::pop_heap(h.begin(), h.end(), std::greater<LW>());
            LW &top = h.back();
            wg_of[i] = top.second;
            load[top.second] += ts[i].c;
            top.first = load[top.second];
            std::push_heap(h.begin(), h.end(), std::greater<LW>());
        }
    };
    // choose g64 (and the 128-wide tiles cut in two) for the smallest makespan
    double best_ms = 1e300;
    int best_g64 = 0, best_h = 0;
    const double w64 = [&] { double w = 0; for (const Tl &t : v64) w += t.c; return w; }();
    const double w128 = [&] { double w = 0; for (const Tl &t : v128) w += t.c; return w; }();
    // candidates: the split that gives each set workgroups in proportion to its load, and one step of 8 either side
    std::vector<int> cands;
    if (v64.empty()) cands.push_back(0);
    else if (v128.empty()) cands.push_back(G);
    else {
        const int c0 = (int)std::lround(G * w64 / (w64 + w128) / 8) * 8;
        for (int c = c0 - 8; c <= c0 + 8; c += 8)
            if (c >= 8 && c <= G - 8) cands.push_back(c);
        if (cands.empty()) cands.push_back(c0 < 8 ? 8 : G - 8);
    }
    auto build = [&](int g64, int h, std::vector<Tl> &a64, std::vector<Tl> &a128) {
        a64 = v64;
        a128.assign(v128.begin(), v128.end() - h);
        for (auto it = v128.end() - h; it != v128.end(); ++it) {   // cut in two 64-wide tiles
            const PkGroup::Prod &p = g.prods[it->p];
            for (int t0 = it->t0; t0 < it->t0 + it->nt; t0 += 64)
                a64.push_back(Tl{it->p, it->rt, t0, std::min(64, it->t0 + it->nt - t0), true, pk_cost(p.nbk, true)});
        }
        (void)g64;
    };
    std::vector<int> seq64, wg64, seq128, wg128;
    for (int g64 : cands) {
        int h = 0;
        if (g64 > 0 && g64 < G && !v128.empty()) {
            const double c128 = v128.back().c, c64 = pk_cost(g.prods[v128.back().p].nbk, true);
            const double hh = (w128 * g64 - w64 * (G - g64)) / (2 * c64 * (G - g64) + c128 * g64);
            h = std::max(0, std::min((int)v128.size(), (int)std::lround(hh)));
        }
        std::vector<Tl> a64, a128;
        build(g64, h, a64, a128);
        if ((!a64.empty() && g64 == 0) || (!a128.empty() && g64 == G)) continue;
        std::vector<double> load(G, 0.0);
        if (!a64.empty()) lpt(a64, 0, g64, seq64, wg64, load);
        if (!a128.empty()) lpt(a128, g64, G - g64, seq128, wg128, load);
        const double ms = *std::max_element(load.begin(), load.end());
        if (ms < best_ms - 1e-9) { best_ms = ms; best_g64 = g64; best_h = h; }
    }
    std::vector<Tl> a64, a128;
    build(best_g64, best_h, a64, a128);
    std::vector<double> load(G, 0.0);
    seq64.clear();
    seq128.clear();
    if (!a64.empty()) lpt(a64, 0, best_g64, seq64, wg64, load);
    if (!a128.empty()) lpt(a128, best_g64, G - best_g64, seq128, wg128, load);
    // each workgroup's tiles in the order they were placed (longest first)
    std::vector<int> cnt(G + 1, 0);
    for (int i : seq64) cnt[wg64[i] + 1]++;
    for (int i : seq128) cnt[wg128[i] + 1]++;
    for (int w = 0; w < G; w++) {
        if (cnt[w + 1] > esq::PK_MAX_TILES) return false;
        cnt[w + 1] += cnt[w];
    }
    std::vector<std::pair<const Tl *, int>> placed(seq64.size() + seq128.size());
    {
        std::vector<int> at(cnt.begin(), cnt.end() - 1);
        for (int i : seq64) placed[at[wg64[i]]++] = {&a64[i], wg64[i]};
        for (int i : seq128) placed[at[wg128[i]]++] = {&a128[i], wg128[i]};
    }
    g.grid = G;
    g.g64 = best_g64;
    g.tiles.clear();
    g.tiles.reserve(placed.size());
    g.wgptr.assign(cnt.begin(), cnt.end());
    for (const auto &pt : placed) {
        const Tl &t = *pt.first;
        const PkGroup::Prod &p = g.prods[t.p];
        const int row0 = p.r0 + esq::MK_ROWS * t.rt;
        esq::PkTile r{};
        r.w = p.W + (size_t)row0 * p.row_bytes;
        r.act = p.act;
        r.y = p.y + (size_t)t.t0 * p.ystride + row0;
        r.astride = p.astride;
        r.ystride4 = 4u * p.ystride;
        r.row_bytes = p.row_bytes;
        r.nbk = p.nbk;
        r.t64 = t.t64 ? 1 : 0;
        r.tok0 = t.t0;
        r.na = p.na;
        r.rows = std::min(esq::MK_ROWS, p.r1 - row0);
        r.ntok = t.nt;
        g.tiles.push_back(r);
    }
    return true;
}

bool mb_eligible(const Req &q) {
    const int mn = g_mb_min.load();
    return (q.type == ES_HIP_Q4_0 || q.type == ES_HIP_Q5_0 || q.type == ES_HIP_Q8_0) && mn > 0 && q.na >= mn && !q.ints &&
           q.r1 > q.r0;
}

bool mq_eligible(const Req &q) {
    const int mn = g_mq_min.load();
    return (q.type == ES_HIP_Q4_K || q.type == ES_HIP_Q2_K) && mn > 0 && q.na >= mn && !q.ints && q.r1 > q.r0;
}

// the pre-pass of q's activations in layout (kind, na_pad), shared with earlier products that read the same ones
const Prep &get_prep(Batch &bt, const Req &q, const FmtInfo &f, int kind, int na_pad) {
    const bool q80 = kind == esq::PREP_KIND_Q80;
    const int nbk = q.cols / (q80 ? 32 : 256);
    const uint64_t astride = q.astride ? q.astride : (uint64_t)nbk * f.ab;
    for (const Prep &p : bt.preps)
        if (p.act == q.act && p.arow == q.arow && p.astride == astride && p.na == q.na && p.nbk == nbk && p.kind == kind &&
            p.na_pad == na_pad)
            return p;
    Prep p{static_cast<const uint8_t *>(q.act), q.arow, astride, q.na, na_pad, nbk, kind, 0, 0};
    p.xq_off = bt.ws_bytes;
    bt.ws_bytes += align256((size_t)nbk * na_pad * (q80 ? 64 : 256));
    p.xm_off = bt.ws_bytes;
    bt.ws_bytes += align256((size_t)nbk * na_pad * (q80 ? 4 : kind ? 36 : 20));   // meta, then the float scales
    bt.preps.push_back(p);
    return bt.preps.back();
}

// Rows per workgroup tile of a batched 32-wide launch (es_hip_mbx.hip): the kernel is VALU-bound per SIMD, so the
// launch's row x activation-tile units are spread over about one workgroup per CU, each job taking its share of the
// workgroups; a tile holds 8 .. MBX_ROWS rows (one to four per wave). Then the tile numbering (with several activation
// tiles, a job's tiles start at a multiple of 8 so that a row tile's activation tiles share an XCD).
void mbx_tiles(MkGroup &g, int cus) {
    double units = 0;
    for (const esq::MkJob &j : g.jobs) units += (double)(j.r1 - j.r0) * j.ntok_tiles;
    g.grid = 0;
    for (esq::MkJob &j : g.jobs) {
        const int rows = j.r1 - j.r0;
        const int wg = std::max(1, (int)((double)cus * rows * j.ntok_tiles / units));
        const int rt = std::max(1, wg / j.ntok_tiles);
        j.rows_per_wg = std::min(esq::MBX_ROWS, std::max(esq::MBX_WAVES, (rows + rt - 1) / rt));
        j.tile0 = g.grid;
        const int row_tiles = (rows + j.rows_per_wg - 1) / j.rows_per_wg;
        g.grid += j.ntok_tiles == 1 ? row_tiles : 8 * ((row_tiles + 7) / 8) * j.ntok_tiles;
    }
}

int plan_batch(const std::vector<Req> &reqs, Batch &bt, bool allow_pk = true) {
    bt = Batch();
    std::vector<Req> mv;
    for (const Req &q : reqs) {
        FmtInfo f;
        if (!fmt_info(q.type, f)) return fail(ES_HIP_EINVAL, "type %u is not computed by this library", q.type);
        if (int rc = check_req(q, f)) return rc;
        if (q.row_bytes) {   // a piece of a long row: the decode kernel carries its chains
            mv.push_back(q);
            continue;
        }
        if (mb_eligible(q)) {   // batched 32-wide: activation groups of at most 64
            const int mm = g_mbm_min.load();   // (the matrix-core kernels address a matrix with 32-bit offsets)
            const bool mfma = mm > 0 && q.na >= mm && (size_t)q.r1 * (q.cols / 32) * f.bb < ((size_t)1 << 31);
            const int nbk32 = q.cols / 32;
            const size_t arows = q.arow ? (size_t)std::max(q.act_rows, 0) : (size_t)q.na;
            const size_t astride = q.astride ? q.astride : (size_t)nbk32 * f.ab;
            if (mfma && g_mbx_on.load() && esq::mbx_nbk_max(nbk32) && (!q.arow || q.act_rows > 0) &&
                arows * astride < ((size_t)1 << 32) - 65536) {
                // the matrix-core kernel reading the Q8_0 rows: rows_per_wg x MBX_TOK tiles, no pre-pass (tiles numbered
                // once the launch's jobs are known, mbx_tiles)
                const int nbkm = esq::mbx_nbk_max(nbk32);
                MkGroup *g = nullptr;
                for (MkGroup &x : bt.mkg)
                    if (x.b32 && x.type == (int)q.type && x.gather == (q.arow != nullptr) && x.nbkm == nbkm) g = &x;
                if (!g) {
                    bt.mkg.push_back(MkGroup{(int)q.type, q.arow != nullptr, nbkm});
                    g = &bt.mkg.back();
                    g->b32 = true;
                }
                esq::MkJob j{};
                j.W = static_cast<const uint8_t *>(q.W);
                j.act = static_cast<const uint8_t *>(q.act);
                j.arow = q.arow;
                j.y = q.y;
                j.astride = astride;
                j.ystride = q.ystride;
                j.row_bytes = (uint64_t)nbk32 * f.bb;
                j.r0 = q.r0;
                j.r1 = q.r1;
                j.cols = q.cols;
                j.na = q.na;
                j.ntok_tiles = (q.na + esq::MBX_TOK - 1) / esq::MBX_TOK;
                g->jobs.push_back(j);
                continue;
            }
            MbGroup *g = nullptr;
            for (MbGroup &x : bt.mbg)
                if (x.type == (int)q.type && x.mfma == mfma) g = &x;
            if (!g) { bt.mbg.push_back(MbGroup{(int)q.type, mfma}); g = &bt.mbg.back(); }
            const int tstep = mfma ? esq::MB32M_TOKENS : 64;
            const Prep *pp = mfma ? &get_prep(bt, q, f, esq::PREP_KIND_Q80, (q.na + 31) / 32 * 32) : nullptr;
            for (int t0 = 0; t0 < q.na; t0 += tstep) {
                int ta = 1;
                while (ta < std::min(64, q.na - t0)) ta <<= 1;
                if (mfma) ta = esq::MB32M_TOKENS;
                esq::MbJob j{};
                j.W = static_cast<const uint8_t *>(q.W);
                j.act = static_cast<const uint8_t *>(q.act);
                j.arow = q.arow;
                if (pp) {   // workspace offsets of this tile's planes until bind()
                    j.xq = reinterpret_cast<const uint8_t *>(pp->xq_off + (size_t)(t0 / 32) * nbk32 * 2048);
                    j.xm = reinterpret_cast<const uint8_t *>(pp->xm_off + (size_t)(t0 / 32) * nbk32 * 128);
                }
                j.y = q.y;
                j.astride = q.astride ? q.astride : (uint64_t)nbk32 * f.ab;
                j.ystride = q.ystride;
                j.row_bytes = (uint64_t)nbk32 * f.bb;
                j.r0 = q.r0;
                j.r1 = q.r1;
                j.cols = q.cols;
                j.na = q.na;
                j.t0 = t0;
                j.ta = ta;
                j.tile0 = g->grid;
                const int rows_per_wg = mfma ? esq::MB32M_ROWS : 4 * (64 / ta);
                g->grid += (q.r1 - q.r0 + rows_per_wg - 1) / rows_per_wg;
                g->jobs.push_back(j);
            }
            continue;
        }
        const int nbk = q.cols / 256;
        if (mx_eligible(q)) {   // one launch per LDS size class; MX_ROWS x MX_TOK tiles
            const int nbkm = esq::mx_nbk_max(nbk);
            MkGroup *g = nullptr;
            const bool gated = q.W2 != nullptr;
            for (MkGroup &x : bt.mkg)
                if (!x.b32 && x.type == (int)q.type && x.gather == (q.arow != nullptr) && x.nbkm == nbkm && x.gated == gated)
                    g = &x;
            if (!g) {
                bt.mkg.push_back(MkGroup{(int)q.type, q.arow != nullptr, nbkm});
                g = &bt.mkg.back();
                g->gated = gated;
            }
            esq::MkJob j{};
            j.W = static_cast<const uint8_t *>(q.W);
            j.W2 = static_cast<const uint8_t *>(q.W2);
            j.act = static_cast<const uint8_t *>(q.act);
            j.arow = q.arow;
            j.y = q.y;
            j.astride = q.astride ? q.astride : (uint64_t)nbk * f.ab;
            j.ystride = gated ? q.ystride : mk_ystride(q);
            j.row_bytes = (uint64_t)nbk * f.bb;
            j.r0 = q.r0;
            j.r1 = q.r1;
            j.cols = q.cols;
            j.na = q.na;
            j.tile0 = g->grid;
            j.ntok_tiles = (q.na + esq::MX_TOK - 1) / esq::MX_TOK;
            const int trows = gated ? 256 : esq::MX_ROWS;   // the gated kernel's tiles are one block of h
            const int row_tiles = (q.r1 - q.r0 + trows - 1) / trows;
            g->grid += j.ntok_tiles == 1 ? row_tiles : 8 * ((row_tiles + 7) / 8) * j.ntok_tiles;
            g->jobs.push_back(j);
            continue;
        }
        if (allow_pk && pk_eligible(q)) {   // the persistent direct kernel: one launch per format, scheduled below
            PkGroup *g = nullptr;
            for (PkGroup &x : bt.pkg)
                if (x.type == (int)q.type) g = &x;
            if (!g) { bt.pkg.push_back(PkGroup{(int)q.type}); g = &bt.pkg.back(); }
            const int nbk = q.cols / 256;
            g->prods.push_back(PkGroup::Prod{static_cast<const uint8_t *>(q.W), static_cast<const uint8_t *>(q.act), q.y,
                                             (uint32_t)(q.astride ? q.astride : (size_t)nbk * 292), (uint32_t)mk_ystride(q),
                                             (uint32_t)((size_t)nbk * f.bb), q.r0, q.r1, nbk, q.na});
            continue;
        }
        if (mk_eligible(q)) {   // one launch per format and tile; MK_ROWS x tok tiles, 8 consecutive ids per row tile group
            const int tok = mk_tok(q);
            MkGroup *g = nullptr;
            for (MkGroup &x : bt.mkg)
                if (!x.b32 && x.type == (int)q.type && x.gather == (q.arow != nullptr) && x.nbkm == 0 && x.tok == tok) g = &x;
            if (!g) {
                bt.mkg.push_back(MkGroup{(int)q.type, q.arow != nullptr});
                g = &bt.mkg.back();
                g->tok = tok;
            }
            esq::MkJob j{};
            j.W = static_cast<const uint8_t *>(q.W);
            j.act = static_cast<const uint8_t *>(q.act);
            j.arow = q.arow;
            j.y = q.y;
            j.astride = q.astride ? q.astride : (uint64_t)nbk * f.ab;
            j.ystride = mk_ystride(q);
            j.row_bytes = (uint64_t)nbk * f.bb;
            j.r0 = q.r0;
            j.r1 = q.r1;
            j.cols = q.cols;
            j.na = q.na;
            j.tile0 = g->grid;
            j.ntok_tiles = (q.na + tok - 1) / tok;
            const int row_tiles = (q.r1 - q.r0 + esq::MK_ROWS - 1) / esq::MK_ROWS;
            g->grid += 8 * ((row_tiles + 7) / 8) * j.ntok_tiles;
            g->jobs.push_back(j);
            continue;
        }
        if (!mm_eligible(q)) {
            if (!mq_eligible(q)) { mv.push_back(q); continue; }
            // small batch: activation groups of at most 64, one launch per (format, 16-wide tiles per group)
            const int na_pad = (q.na + 15) / 16 * 16;
            const Prep &pp = get_prep(bt, q, f, q.type == ES_HIP_Q4_K ? 0 : 1, na_pad);
            for (int t0 = 0; t0 < q.na; t0 += 64) {
                const int wn = (std::min(64, q.na - t0) + 15) / 16;
                MqGroup *g = nullptr;
                for (MqGroup &x : bt.mqg)
                    if (x.type == (int)q.type && x.wn == wn) g = &x;
                if (!g) { bt.mqg.push_back(MqGroup{(int)q.type, wn}); g = &bt.mqg.back(); }
                esq::MqJob j{};
                j.W = static_cast<const uint8_t *>(q.W);
                j.xq = reinterpret_cast<const uint8_t *>(pp.xq_off);
                j.xm = reinterpret_cast<const uint8_t *>(pp.xm_off);
                j.y = q.y;
                j.ystride = q.ystride;
                j.row_bytes = (uint64_t)nbk * f.bb;
                j.r0 = q.r0;
                j.r1 = q.r1;
                j.cols = q.cols;
                j.na = q.na;
                j.na_pad = na_pad;
                j.t0 = t0;
                j.tile0 = g->grid;
                g->grid += (q.r1 - q.r0 + 63) / 64;
                g->jobs.push_back(j);
            }
            continue;
        }
        const int pad = q.type == ES_HIP_Q4_K ? esq::MM_NA_PAD : 64;
        // Q2_K batches of up to 32 share one 32-wide tile: few launches for MoE experts of any size
        const int na_pad = q.na <= 16 && q.type != ES_HIP_Q2_K ? 16 : q.na <= 32 ? 32 : q.na <= 64 ? 64 : (q.na + pad - 1) / pad * pad;
        const Prep *pp = &get_prep(bt, q, f, 2, na_pad);
        esq::MmJob j{};
        j.W = static_cast<const uint8_t *>(q.W);
        j.xq = reinterpret_cast<const uint8_t *>(pp->xq_off);
        j.xm = reinterpret_cast<const uint8_t *>(pp->xm_off);
        j.y = q.y;
        j.ystride = q.ystride;
        j.row_bytes = (uint64_t)nbk * f.bb;
        j.r0 = q.r0;
        j.r1 = q.r1;
        j.cols = q.cols;
        j.na = q.na;
        j.na_pad = na_pad;
        bt.mm.push_back({(int)q.type, j});
    }
    // one launch per tile shape; inside a launch the longest rows (most superblocks) come first, so the longest-running
    // workgroups start first
    std::stable_sort(bt.mm.begin(), bt.mm.end(),
                     [](const std::pair<int, esq::MmJob> &x, const std::pair<int, esq::MmJob> &y) { return x.second.cols > y.second.cols; });
    for (auto [type, j] : bt.mm) {
        int bm, bn, nw;
        mm_tile(type, j, bm, bn, nw);
        MmGroup *g = nullptr;
        for (MmGroup &x : bt.mmg)
            if (x.type == type && x.bm == bm && x.bn == bn && x.nw == nw) g = &x;
        if (!g) { bt.mmg.push_back(MmGroup{type, bm, bn, nw}); g = &bt.mmg.back(); }
        j.tile0 = g->grid;   // a multiple of 8: the kernel maps tiles to XCDs by id % 8
        j.ntok_tiles = j.na_pad / bn;
        const int row_tiles = (j.r1 - j.r0 + bm - 1) / bm;
        g->grid += 8 * ((row_tiles + 7) / 8) * j.ntok_tiles;
        g->jobs.push_back(j);
    }
    for (MkGroup &g : bt.mkg)
        if (g.b32) mbx_tiles(g, device().cus);
    for (PkGroup &g : bt.pkg)
        if (!pk_schedule(g, device().cus)) return plan_batch(reqs, bt, false);   // too many tiles for one launch
    // a pre-pass numbers its 16-byte items with 32-bit indices
    for (const Prep &p : bt.preps)
        if ((long)p.na_pad * p.nbk * esq::prep_words(p.kind) > (1L << 30))
            return fail(ES_HIP_EINVAL, "%d activations of %d blocks: above 2^30 pre-pass items per product", p.na, p.nbk);
    if (int rc = plan_groups(mv, bt.mv)) return rc;
    size_t off = 0;
    for (const Group &g : bt.mv) {
        bt.mv_off.push_back(off);
        off += align256(g.jobs.size() * sizeof(MvJob));
    }
    for (PkGroup &g : bt.pkg) {
        g.off = off;
        off += align256(g.tiles.size() * sizeof(esq::PkTile)) + align256(g.wgptr.size() * sizeof(int));
    }
    for (MmGroup &g : bt.mmg) {
        g.off = off;
        off += align256(g.jobs.size() * sizeof(esq::MmJob));
    }
    for (MkGroup &g : bt.mkg) {
        g.off = off;
        off += align256(g.jobs.size() * sizeof(esq::MkJob));
    }
    for (MqGroup &g : bt.mqg) {
        g.off = off;
        off += align256(g.jobs.size() * sizeof(esq::MqJob));
    }
    for (MbGroup &g : bt.mbg) {
        g.off = off;
        off += align256(g.jobs.size() * sizeof(esq::MbJob));
    }
    bt.prep_off = off;
    off += align256(bt.preps.size() * sizeof(esq::PrepJob));
    bt.table_bytes = off;
    return ES_HIP_OK;
}

// point the matrix-core jobs at a workspace of ws_bytes
void bind(Batch &bt, uint8_t *ws) {
    for (MmGroup &g : bt.mmg)
        for (esq::MmJob &j : g.jobs) {
            j.xq = ws + reinterpret_cast<uintptr_t>(j.xq);
            j.xm = ws + reinterpret_cast<uintptr_t>(j.xm);
        }
    for (MqGroup &g : bt.mqg)
        for (esq::MqJob &j : g.jobs) {
            j.xq = ws + reinterpret_cast<uintptr_t>(j.xq);
            j.xm = ws + reinterpret_cast<uintptr_t>(j.xm);
        }
    for (MbGroup &g : bt.mbg)
        if (g.mfma)
            for (esq::MbJob &j : g.jobs) {
                j.xq = ws + reinterpret_cast<uintptr_t>(j.xq);
                j.xm = ws + reinterpret_cast<uintptr_t>(j.xm);
            }
    bt.pj.clear();
    bt.prep_total = 0;
    for (Prep &p : bt.preps) {   // offsets become addresses too (kept as integers)
        p.xq_off = reinterpret_cast<uintptr_t>(ws) + p.xq_off;
        p.xm_off = reinterpret_cast<uintptr_t>(ws) + p.xm_off;
        esq::PrepJob j{p.act, p.arow, reinterpret_cast<uint8_t *>(p.xq_off), reinterpret_cast<uint8_t *>(p.xm_off), p.astride,
                       bt.prep_total, p.na, p.na_pad, p.nbk, p.kind};
        bt.pj.push_back(j);
        const long n = (long)p.na_pad * p.nbk * esq::prep_words(p.kind);
        bt.prep_total += (n + esq::PREP_SPAN - 1) / esq::PREP_SPAN * esq::PREP_SPAN;
    }
}

std::vector<uint8_t> table_image(const Batch &bt) {
    std::vector<uint8_t> img(bt.table_bytes);
    for (size_t i = 0; i < bt.mv.size(); i++)
        memcpy(img.data() + bt.mv_off[i], bt.mv[i].jobs.data(), bt.mv[i].jobs.size() * sizeof(MvJob));
    for (const MmGroup &g : bt.mmg) memcpy(img.data() + g.off, g.jobs.data(), g.jobs.size() * sizeof(esq::MmJob));
    for (const MkGroup &g : bt.mkg) memcpy(img.data() + g.off, g.jobs.data(), g.jobs.size() * sizeof(esq::MkJob));
    for (const PkGroup &g : bt.pkg) {
        memcpy(img.data() + g.off, g.tiles.data(), g.tiles.size() * sizeof(esq::PkTile));
        memcpy(img.data() + g.off + align256(g.tiles.size() * sizeof(esq::PkTile)), g.wgptr.data(), g.wgptr.size() * sizeof(int));
    }
    for (const MqGroup &g : bt.mqg) memcpy(img.data() + g.off, g.jobs.data(), g.jobs.size() * sizeof(esq::MqJob));
    for (const MbGroup &g : bt.mbg) memcpy(img.data() + g.off, g.jobs.data(), g.jobs.size() * sizeof(esq::MbJob));
    if (!bt.pj.empty()) memcpy(img.data() + bt.prep_off, bt.pj.data(), bt.pj.size() * sizeof(esq::PrepJob));
    return img;
}

// launches in stream order: pre-passes, decode kernels, matrix-core kernel. tables: the uploaded image, or null to pass
// single jobs by value.
int launch_batch(const Batch &bt, const uint8_t *tables, int order, hipStream_t s) {
    hipError_t e;
    if (tables && bt.pj.size() > 1) {   // every pre-pass in one launch (a single one goes by value: no table read first)
        e = esq::prep_launch(reinterpret_cast<const esq::PrepJob *>(tables + bt.prep_off), (int)bt.pj.size(), bt.pj[0],
                             bt.prep_total, s);
        if (e != hipSuccess) return hip_fail(e, "pre-pass launch");
    } else {
        for (esq::PrepJob j : bt.pj) {
            const long n = (long)j.na_pad * j.nbk * esq::prep_words(j.kind);
            j.start = 0;
            if ((e = esq::prep_launch(nullptr, 1, j, n, s)) != hipSuccess) return hip_fail(e, "pre-pass launch");
        }
    }
    for (size_t i = 0; i < bt.mv.size(); i++) {
        const Group &g = bt.mv[i];
        const MvJob *dj = tables ? reinterpret_cast<const MvJob *>(tables + bt.mv_off[i]) : nullptr;
        if ((e = esq::mv_launch(g.L, dj, (int)g.jobs.size(), g.jobs[0], order, s)) != hipSuccess) return hip_fail(e, "kernel launch");
    }
    for (const MmGroup &g : bt.mmg) {
        const esq::MmJob *dj = tables ? reinterpret_cast<const esq::MmJob *>(tables + g.off) : nullptr;
        if ((e = esq::mm_launch(g.type, g.bm, g.bn, g.nw, dj, (int)g.jobs.size(), g.jobs[0], g.grid, order, s, g.jobs.data())) !=
            hipSuccess)
            return hip_fail(e, "matrix-core launch");
    }
    for (const PkGroup &g : bt.pkg) {   // (always from the uploaded tables)
        if (!tables) return fail(ES_HIP_EINVAL, "the persistent kernel needs its tile tables on the device");
        const esq::PkTile *tl = reinterpret_cast<const esq::PkTile *>(tables + g.off);
        const int *wp = reinterpret_cast<const int *>(tables + g.off + align256(g.tiles.size() * sizeof(esq::PkTile)));
        if ((e = g.ws ? esq::ws_launch(g.type, tl, wp, g.grid, order, s) : esq::pk_launch(g.type, tl, wp, g.grid, g.g64, order, s)) !=
            hipSuccess)
            return hip_fail(e, "matrix-core launch");
    }
    for (const MkGroup &g : bt.mkg) {
        const esq::MkJob *dj = tables ? reinterpret_cast<const esq::MkJob *>(tables + g.off) : nullptr;
        if ((e = g.b32    ? esq::mbx_launch(g.type, g.gather, g.nbkm, dj, (int)g.jobs.size(), g.jobs[0], g.grid, order, s)
                 : g.nbkm && g.gated ? esq::mxg_launch(g.gather, g.nbkm, dj, (int)g.jobs.size(), g.jobs[0], g.grid, order, s)
                 : g.nbkm ? esq::mx_launch(g.type, g.gather, g.nbkm, dj, (int)g.jobs.size(), g.jobs[0], g.grid, order, s)
                          : esq::mk_launch(g.type, g.gather, g.tok, dj, (int)g.jobs.size(), g.jobs[0], g.grid, order, s)) !=
            hipSuccess)
            return hip_fail(e, "matrix-core launch");
    }
    for (const MbGroup &g : bt.mbg) {
        const esq::MbJob *dj = tables ? reinterpret_cast<const esq::MbJob *>(tables + g.off) : nullptr;
        if ((e = (g.mfma ? esq::mb32m_launch : esq::mb32_launch)(g.type, dj, (int)g.jobs.size(), g.jobs[0], g.grid, order, s)) !=
            hipSuccess)
            return hip_fail(e, "batched launch");
    }
    for (const MqGroup &g : bt.mqg) {
        const esq::MqJob *dj = tables ? reinterpret_cast<const esq::MqJob *>(tables + g.off) : nullptr;
        if ((e = esq::mq_launch(g.type, g.wn, dj, (int)g.jobs.size(), g.jobs[0], g.grid, order, s)) != hipSuccess)
            return hip_fail(e, "small-batch launch");
    }
    return ES_HIP_OK;
}

// ---- reusable device scratch (host drop-ins, run_jobs tables) ----------------------------------------------------
struct Scratch {
    std::mutex mu;
    void *p = nullptr;
    size_t n = 0;
    int get(size_t bytes, void **out) {
        if (bytes > n) {
            if (p) (void)hipFree(p);
            p = nullptr;
            n = 0;
            size_t want = std::max(bytes, (size_t)1 << 20);
            hipError_t e = hipMalloc(&p, want);
            if (e != hipSuccess) return hip_fail(e, "hipMalloc scratch");
            n = want;
        }
        *out = p;
        return ES_HIP_OK;
    }
};
Scratch g_table, g_wtmp, g_atmp, g_ytmp;
std::mutex g_call_mu;   // serialises the synchronous convenience entry points that share scratch

// ---- page-locked host staging for the entry points on host memory ----------------------------------------------------
// Activations are packed here before one copy up and outputs land here before they are spread to the caller's arrays:
// copies from and to page-locked memory run at the link's rate, and the buffers persist, so a call neither allocates nor
// faults in fresh pages. Used under g_call_mu.
struct HostStage {
    void *p = nullptr;
    size_t n = 0;
    int get(size_t bytes, void **out) {
        if (bytes > n) {
            if (p) (void)hipHostFree(p);
            p = nullptr;
            n = 0;
            const size_t want = std::max(bytes, (size_t)1 << 20);
            hipError_t e = hipHostMalloc(&p, want, hipHostMallocDefault);
            if (e != hipSuccess) return hip_fail(e, "hipHostMalloc staging");
            n = want;
        }
        *out = p;
        return ES_HIP_OK;
    }
};
HostStage g_hin, g_hout;

// The host-to-host copies of one call (packing activations, spreading outputs), over up to 8 threads when they add up to
// more than 8 MB: a prefill-sized queue returns tens of MB of outputs, which one core copies at a fraction of the link's rate.
struct HCopy {
    void *dst;
    const void *src;
    size_t bytes;
};
void host_copies(const std::vector<HCopy> &v) {
    size_t total = 0;
    for (const HCopy &c : v) total += c.bytes;
    const unsigned nt = std::min(8u, std::max(1u, std::thread::hardware_concurrency()));
    auto run = [](const std::vector<HCopy> &w) { for (const HCopy &c : w) memcpy(c.dst, c.src, c.bytes); };
    if (total < ((size_t)8 << 20) || nt == 1) return run(v);
    const size_t piece = (total + nt - 1) / nt;   // each thread takes a contiguous share of about total / nt bytes
    std::vector<std::vector<HCopy>> work(nt);
    size_t acc = 0;
    for (HCopy c : v)
        while (c.bytes) {
            const unsigned w = (unsigned)std::min<size_t>(acc / piece, nt - 1);
            const size_t b = w == nt - 1 ? c.bytes : std::min(c.bytes, (w + 1) * piece - acc);
            work[w].push_back({c.dst, c.src, b});
            c.dst = static_cast<uint8_t *>(c.dst) + b;
            c.src = static_cast<const uint8_t *>(c.src) + b;
            c.bytes -= b;
            acc += b;
        }
    std::vector<std::thread> th;
    try {
        for (unsigned w = 1; w < nt; w++) th.emplace_back(run, std::cref(work[w]));
    } catch (...) {   // no thread to be had: the remaining shares run here
        for (unsigned w = 1 + (unsigned)th.size(); w < nt; w++) run(work[w]);
    }
    run(work[0]);
    for (std::thread &t : th) t.join();
}

// ---- weight registry ------------------------------------------------------------------------------------------------
struct Reg {
    size_t bytes;
    void *dev;
};
std::mutex g_reg_mu;
std::map<uintptr_t, Reg> g_reg;

// device address of host range [h, h + n) if it lies inside one registered range
void *reg_lookup(const void *h, size_t n) {
    std::lock_guard<std::mutex> lk(g_reg_mu);
    const uintptr_t a = reinterpret_cast<uintptr_t>(h);
    auto it = g_reg.upper_bound(a);
    if (it == g_reg.begin()) return nullptr;
    --it;
    if (a + n > it->first + it->second.bytes) return nullptr;
    return static_cast<uint8_t *>(it->second.dev) + (a - it->first);
}

// Batches without a pre-pass workspace are kept after their first call, tables on the device: the engine repeats the same
// products on the same buffers at every step (dense_n's gate/up and down per layer), and a repeat then launches from the
// kept tables with no planning and no upload. Such tables are read-only, so every stream may share them. The key is every
// request field and the planning settings' generation; at most BC_MAX batches are kept, the least recently used one freed
// first (hipFree waits for kernels that may still read it).
struct CachedBatch {
    std::vector<Req> reqs;
    uint64_t gen, tick;
    Batch bt;
    void *dev;
};
constexpr size_t BC_MAX = 64;
std::mutex g_bc_mu;
std::vector<CachedBatch> g_bc;
uint64_t g_bc_tick = 0;

bool same_reqs(const std::vector<Req> &a, const std::vector<Req> &b) {
    if (a.size() != b.size()) return false;
    for (size_t i = 0; i < a.size(); i++) {
        const Req &x = a[i], &y = b[i];
        if (x.type != y.type || x.W != y.W || x.act != y.act || x.y != y.y || x.ints != y.ints || x.aux != y.aux ||
            x.r0 != y.r0 || x.r1 != y.r1 || x.cols != y.cols || x.na != y.na || x.astride != y.astride ||
            x.ystride != y.ystride || x.arow != y.arow || x.act_rows != y.act_rows || x.row_bytes != y.row_bytes ||
            x.chain != y.chain || x.lanes != y.lanes)
            return false;
    }
    return true;
}

// A kept batch for reqs, launched on s: 1 if launched (rc set), 0 if none is kept.
bool has_pieces(const std::vector<Req> &reqs) {
    for (const Req &q : reqs)
        if (q.row_bytes) return true;
    return false;
}

int cached_launch(const std::vector<Req> &reqs, hipStream_t s, int order, int &rc) {
    if (has_pieces(reqs)) return 0;   // pieces of a call's long rows are planned each time (their lane chains are per call)
    const uint64_t gen = g_cfg_gen.load();
    std::lock_guard<std::mutex> lk(g_bc_mu);
    for (CachedBatch &c : g_bc)
        if (c.gen == gen && same_reqs(c.reqs, reqs)) {
            c.tick = ++g_bc_tick;
            rc = launch_batch(c.bt, static_cast<const uint8_t *>(c.dev), order >= 0 ? order : g_order.load(), s);
            return 1;
        }
    return 0;
}

// Keeps a planned batch without a pre-pass workspace and launches it on s: 1 if kept (rc set), 0 if it cannot be kept.
int keep_and_launch(const std::vector<Req> &reqs, Batch &bt, hipStream_t s, int order, int &rc) {
    if (bt.ws_bytes != 0 || bt.table_bytes == 0 || has_pieces(reqs)) return 0;
    const uint64_t gen = g_cfg_gen.load();
    void *dev = nullptr;
    hipError_t e = hipMalloc(&dev, bt.table_bytes);
    if (e != hipSuccess) { rc = hip_fail(e, "hipMalloc (kept job tables)"); return 1; }
    bind(bt, static_cast<uint8_t *>(dev) + align256(bt.table_bytes));
    const std::vector<uint8_t> img = table_image(bt);
    // the upload is complete before any stream may launch from the tables
    if ((e = hipMemcpy(dev, img.data(), img.size(), hipMemcpyHostToDevice)) != hipSuccess ||
        (e = hipDeviceSynchronize()) != hipSuccess) {
        (void)hipFree(dev);
        rc = hip_fail(e, "job table upload");
        return 1;
    }
    std::lock_guard<std::mutex> lk(g_bc_mu);
    if (g_bc.size() >= BC_MAX) {
        auto lru = std::min_element(g_bc.begin(), g_bc.end(), [](const CachedBatch &a, const CachedBatch &b) { return a.tick < b.tick; });
        (void)hipFree(lru->dev);
        g_bc.erase(lru);
    }
    g_bc.push_back(CachedBatch{reqs, gen, ++g_bc_tick, std::move(bt), dev});
    rc = launch_batch(g_bc.back().bt, static_cast<const uint8_t *>(dev), order >= 0 ? order : g_order.load(), s);
    return 1;
}

// Plan, upload the job tables (and bind the pre-pass workspace) in scratch, launch: the path shared by run_jobs,
// run_jobs_host and the host drop-ins. The caller holds g_call_mu. The tables go up from page-locked staging, stream-ordered
// behind the caller's earlier work on s; every call waits for its kernels before it returns (with sync here, or, for the
// host entry points, after their output copy), so no earlier call's kernels still read the scratch. A call that failed
// between its first copy or launch and that wait leaves g_table_pending set, and the next call first waits for the device.
HostStage g_htab;
bool g_table_pending = false;

int settle() {   // before the staging or the scratch is reused: the wait a failed call skipped
    if (!g_table_pending) return ES_HIP_OK;
    hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return hip_fail(e, "hipDeviceSynchronize");
    g_table_pending = false;
    return ES_HIP_OK;
}

// Rows longer than ES_HIP_MAX_COLS_* (one row's float terms no longer fit a workgroup's LDS) run as column pieces of at
// most that many columns, one batch per piece in stream order, each piece continuing the chains where the one before
// stopped: es_matvec's sums over a row's blocks (src/es_quant.c:1852-1945, per format at :1013-1117 and :1252-1469)
// are sequential in block order, and the pieces cut them at block boundaries, so every output is the whole row's. A
// K-quant row (and a 32-element row in the scalar order) carries its one chain in y; the AVX2 order of the 32-element
// formats carries eight lane chains per output in a stream-ordered allocation. Phase 0 holds every other product and the
// first piece of each long one; phase p the p-th pieces.
bool has_long(const std::vector<Req> &reqs) {
    for (const Req &q : reqs) {
        FmtInfo f;
        if (!q.row_bytes && !q.ints && fmt_info(q.type, f) && q.cols > (f.be == 32 ? ES_HIP_MAX_COLS_32 : ES_HIP_MAX_COLS_256))
            return true;
    }
    return false;
}

// checks every long request (before anything is allocated or launched) and counts the floats of its lane chains
int count_lanes(const std::vector<Req> &reqs, int order, size_t &nlanes) {
    const bool x86 = order != ES_HIP_ORDER_SCALAR;
    nlanes = 0;
    for (const Req &q : reqs) {
        FmtInfo f;
        if (!fmt_info(q.type, f)) return fail(ES_HIP_EINVAL, "type %u is not computed by this library", q.type);
        if (q.ints || q.cols <= (f.be == 32 ? ES_HIP_MAX_COLS_32 : ES_HIP_MAX_COLS_256)) continue;
        if (int rc = check_req(q, f, false)) return rc;
        if (f.be == 32 && x86 && q.r1 > q.r0 && q.na > 0) nlanes += (size_t)q.na * (q.r1 - q.r0) * 8;
    }
    return ES_HIP_OK;
}

// the phases of reqs (after count_lanes), lane chains in lanes
void cut_pieces(const std::vector<Req> &reqs, int order, float *lanes, std::vector<std::vector<Req>> &phases) {
    const bool x86 = order != ES_HIP_ORDER_SCALAR;
    phases.assign(1, {});
    size_t lo = 0;
    for (const Req &q : reqs) {
        FmtInfo f;
        fmt_info(q.type, f);
        const int cmax = f.be == 32 ? ES_HIP_MAX_COLS_32 : ES_HIP_MAX_COLS_256;
        if (q.ints || q.cols <= cmax || q.r1 == q.r0 || q.na == 0) {
            phases[0].push_back(q);
            continue;
        }
        const int nbk = q.cols / f.be, pb = cmax / f.be, np = (nbk + pb - 1) / pb;
        float *ql = f.be == 32 && x86 ? lanes + lo : nullptr;
        if (ql) lo += (size_t)q.na * (q.r1 - q.r0) * 8;
        for (int p = 0; p < np; p++) {
            const int b0 = p * pb, b1 = std::min(nbk, b0 + pb);
            Req r = q;
            r.W = static_cast<const uint8_t *>(q.W) + (size_t)b0 * f.bb;
            r.act = static_cast<const uint8_t *>(q.act) + (size_t)b0 * f.ab;
            r.cols = (b1 - b0) * f.be;
            r.astride = q.astride ? q.astride : (size_t)nbk * f.ab;
            r.row_bytes = (size_t)nbk * f.bb;
            r.chain = (p > 0 ? esq::MV_CHAIN_IN : 0) | (ql && p + 1 < np ? esq::MV_CHAIN_LANES_OUT : 0);
            r.lanes = ql;
            if ((int)phases.size() <= p) phases.resize(p + 1);
            phases[p].push_back(r);
        }
    }
}

template <typename RUN> int run_in_pieces(const std::vector<Req> &reqs, hipStream_t s, int order, RUN run) {
    size_t nlanes = 0;
    if (int rc = count_lanes(reqs, order, nlanes)) return rc;
    float *lanes = nullptr;
    if (nlanes) {
        hipError_t e = hipMallocAsync(reinterpret_cast<void **>(&lanes), nlanes * sizeof(float), s);
        if (e != hipSuccess) return hip_fail(e, "hipMallocAsync (lane chains of long rows)");
    }
    std::vector<std::vector<Req>> phases;
    cut_pieces(reqs, order, lanes, phases);
    int rc = ES_HIP_OK;
    for (const std::vector<Req> &ph : phases)
        if (!rc && !ph.empty()) rc = run(ph, order);
    if (lanes) {
        hipError_t e = hipFreeAsync(lanes, s);
        if (!rc && e != hipSuccess) rc = hip_fail(e, "hipFreeAsync");
    }
    return rc;
}

int run_launch(const std::vector<Req> &reqs, hipStream_t s, int order) {   // order -1: es_hip_set_order's
    if (has_long(reqs))
        return run_in_pieces(reqs, s, order >= 0 ? order : g_order.load(),
                             [&](const std::vector<Req> &ph, int o) { return run_launch(ph, s, o); });
    int rc = ES_HIP_OK;
    if (cached_launch(reqs, s, order, rc)) {
        if (!rc) g_table_pending = true;   // the caller's wait follows
        return rc;
    }
    Batch bt;
    if (int e = plan_batch(reqs, bt)) return e;
    if (bt.mv.empty() && bt.mm.empty() && bt.mqg.empty() && bt.mbg.empty() && bt.mkg.empty() && bt.pkg.empty()) return ES_HIP_OK;
    if (int e = settle()) return e;
    if (keep_and_launch(reqs, bt, s, order, rc)) {
        g_table_pending = true;
        return rc;
    }
    hipError_t e;
    void *dev = nullptr, *htab = nullptr;
    const size_t ws_at = align256(bt.table_bytes);
    if (int rc = g_table.get(ws_at + bt.ws_bytes, &dev)) return rc;
    bind(bt, static_cast<uint8_t *>(dev) + ws_at);
    const std::vector<uint8_t> img = table_image(bt);
    if (!img.empty()) {
        if (int rc = g_htab.get(img.size(), &htab)) return rc;
        memcpy(htab, img.data(), img.size());
        g_table_pending = true;
        if ((e = hipMemcpyAsync(dev, htab, img.size(), hipMemcpyHostToDevice, s)) != hipSuccess) return hip_fail(e, "job table upload");
    }
    g_table_pending = true;
    return launch_batch(bt, static_cast<const uint8_t *>(dev), order >= 0 ? order : g_order.load(), s);
}

// the caller's wait after run_launch (and whatever it queued behind it on s)
int finish(hipStream_t s) {
    hipError_t e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
    g_table_pending = false;
    return ES_HIP_OK;
}

// run_launch and wait: like the reference's run_jobs, every product is done on return
int run_sync(const std::vector<Req> &reqs, hipStream_t s, int order = -1) {
    if (int rc = run_launch(reqs, s, order)) return rc;
    return finish(s);
}

}  // namespace

// =====================================================================================================================
extern "C" {

int es_hip_available(void) { return need_device() == ES_HIP_OK ? 1 : 0; }
const char *es_hip_last_error(void) { return g_err.c_str(); }
const char *es_hip_device_name(void) { return device().arch.c_str(); }

int es_hip_set_order(int order) {
    if (order < ES_HIP_ORDER_X86_CONTRACT || order > ES_HIP_ORDER_SCALAR) return fail(ES_HIP_EINVAL, "bad order %d", order);
    return g_order.exchange(order);
}
int es_hip_get_order(void) { return g_order.load(); }

int es_hip_quant_supported(uint32_t type) {
    FmtInfo f;
    return fmt_info(type, f) ? 1 : 0;
}

size_t es_hip_row_bytes(uint32_t type, int cols) {
    FmtInfo f;
    if (!fmt_info(type, f) || cols < 0) return 0;
    return (size_t)(cols / f.be) * f.bb;   // src/es_quant.c:39-73: whole blocks
}

// ---- memory helpers ---------------------------------------------------------------------------------------------------
void *es_hip_malloc(size_t bytes) {
    if (need_device()) return nullptr;
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
    if (e != hipSuccess) { hip_fail(e, "hipMalloc"); return nullptr; }
    return p;
}
int es_hip_free(void *dev) {
    if (!dev) return ES_HIP_OK;
    hipError_t e = hipFree(dev);
    return e == hipSuccess ? ES_HIP_OK : hip_fail(e, "hipFree");
}
void *es_hip_host_alloc(size_t bytes) {
    if (need_device()) return nullptr;
    void *p = nullptr;
    hipError_t e = hipHostMalloc(&p, bytes ? bytes : 1, hipHostMallocDefault);
    if (e != hipSuccess) { hip_fail(e, "hipHostMalloc"); return nullptr; }
    return p;
}
int es_hip_host_free(void *host) {
    if (!host) return ES_HIP_OK;
    hipError_t e = hipHostFree(host);
    return e == hipSuccess ? ES_HIP_OK : hip_fail(e, "hipHostFree");
}
int es_hip_memcpy_h2d(void *dev, const void *host, size_t bytes) {
    if (int rc = need_device()) return rc;
    hipError_t e = hipMemcpy(dev, host, bytes, hipMemcpyHostToDevice);
    return e == hipSuccess ? ES_HIP_OK : hip_fail(e, "hipMemcpy H2D");
}
int es_hip_memcpy_d2h(void *host, const void *dev, size_t bytes) {
    if (int rc = need_device()) return rc;
    hipError_t e = hipMemcpy(host, dev, bytes, hipMemcpyDeviceToHost);
    return e == hipSuccess ? ES_HIP_OK : hip_fail(e, "hipMemcpy D2H");
}
int es_hip_memcpy_d2d(void *dst, const void *src, size_t bytes) {
    if (int rc = need_device()) return rc;
    hipError_t e = hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice);
    return e == hipSuccess ? ES_HIP_OK : hip_fail(e, "hipMemcpy D2D");
}
int es_hip_memset(void *dev, int value, size_t bytes) {
    if (int rc = need_device()) return rc;
    hipError_t e = hipMemset(dev, value, bytes);
    return e == hipSuccess ? ES_HIP_OK : hip_fail(e, "hipMemset");
}
int es_hip_synchronize(void) {
    if (int rc = need_device()) return rc;
    hipError_t e = hipDeviceSynchronize();
    return e == hipSuccess ? ES_HIP_OK : hip_fail(e, "hipDeviceSynchronize");
}

// ---- products on device memory ----------------------------------------------------------------------------------------
// Plan and launch a batch in stream order: a single decode job by value; anything else (several jobs per launch,
// pre-passes) with a stream-ordered allocation for the job tables and the pre-pass workspace, freed in stream order. The
// tables are copied from pageable memory, which the copy has consumed when it returns.
static int run_async(const std::vector<Req> &reqs, hipStream_t s, int order = -1) {
    if (has_long(reqs))
        return run_in_pieces(reqs, s, order >= 0 ? order : g_order.load(),
                             [&](const std::vector<Req> &ph, int o) { return run_async(ph, s, o); });
    int rc = ES_HIP_OK;
    if (cached_launch(reqs, s, order, rc)) return rc;
    Batch bt;
    if (int e = plan_batch(reqs, bt)) return e;
    if (bt.mm.empty() && bt.mqg.empty() && bt.mbg.empty() && bt.mkg.empty() && bt.pkg.empty() && bt.mv.size() <= 1 &&
        (bt.mv.empty() || bt.mv[0].jobs.size() == 1))
        return bt.mv.empty() ? ES_HIP_OK : launch_single(bt.mv[0], s, order);
    if (keep_and_launch(reqs, bt, s, order, rc)) return rc;
    void *dev = nullptr;
    const size_t ws_at = align256(bt.table_bytes);
    hipError_t e = hipMallocAsync(&dev, std::max<size_t>(ws_at + bt.ws_bytes, 256), s);
    if (e != hipSuccess) return hip_fail(e, "hipMallocAsync (tables and workspace)");
    bind(bt, static_cast<uint8_t *>(dev) + ws_at);
    const std::vector<uint8_t> img = table_image(bt);
    if (!img.empty() && (e = hipMemcpyAsync(dev, img.data(), img.size(), hipMemcpyHostToDevice, s)) != hipSuccess)
        rc = hip_fail(e, "job table upload");
    if (!rc) rc = launch_batch(bt, static_cast<const uint8_t *>(dev), order >= 0 ? order : g_order.load(), s);
    e = hipFreeAsync(dev, s);
    if (rc) return rc;
    return e == hipSuccess ? ES_HIP_OK : hip_fail(e, "hipFreeAsync");
}

int es_hip_matvec_multi_dev(uint32_t type, const void *W, int cols, int r0, int r1, const void *act, size_t astride, int na,
                            float *y, size_t ystride, void *stream) {
    if (int rc = need_device()) return rc;
    return run_async({{type, W, act, y, nullptr, nullptr, r0, r1, cols, na, astride, ystride}}, static_cast<hipStream_t>(stream));
}

// dense_n (src/es_engine.c:957-972): gate and up into the engine's [token][2 ff] rows in one batch, SwiGLU fused with the
// preparation of h for the down product's activation kind, then down.
int es_hip_dense_ffn_dev(uint32_t gate_type, const void *wg, uint32_t up_type, const void *wu, uint32_t down_type,
                         const void *wd, int n, int ff, int N, const void *x, size_t xstride, float *gu, void *hq,
                         float *out, size_t ostride, void *stream) {
    if (int rc = need_device()) return rc;
    FmtInfo fg, fu, fd;
    if (!fmt_info(gate_type, fg) || !fmt_info(up_type, fu) || !fmt_info(down_type, fd))
        return fail(ES_HIP_EINVAL, "a weight type is not computed by this library");
    if (fg.ab != fu.ab) return fail(ES_HIP_EINVAL, "gate and up must take the same kind of activation blocks");
    if (n <= 0 || ff <= 0 || N < 0) return fail(ES_HIP_EINVAL, "bad shape n %d ff %d N %d", n, ff, N);
    const bool dq8k = fd.ab == 292;   // K-quant down: Q8_K activations; Q4_0/Q5_0/Q8_0: Q8_0
    if (ff % (dq8k ? 256 : 32)) return fail(ES_HIP_EINVAL, "ff %d is not a whole number of the down type's blocks", ff);
    if (N == 0) return ES_HIP_OK;
    if (!wg || !wu || !wd || !x || !gu || !hq || !out) return fail(ES_HIP_EINVAL, "null pointer");
    if (ostride < (size_t)n) return fail(ES_HIP_EINVAL, "ostride %zu < n %d", ostride, n);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const size_t gus = 2 * (size_t)ff;
    if (int rc = run_async({{gate_type, wg, x, gu, nullptr, nullptr, 0, ff, n, N, xstride, gus},
                            {up_type, wu, x, gu + ff, nullptr, nullptr, 0, ff, n, N, xstride, gus}}, s))
        return rc;
    const size_t hs = (size_t)(ff / (dq8k ? 256 : 32)) * fd.ab;   // packed activation blocks of h, per token
    if (int rc = es_hip_swiglu_prepare_dev(gu, gus, N, ff, nullptr, 0, dq8k ? nullptr : hq, hs, dq8k ? hq : nullptr, hs, stream))
        return rc;
    return run_async({{down_type, wd, hq, out, nullptr, nullptr, 0, n, ff, N, hs, ostride}}, s);
}

// ---- the product entry point that allocates nothing ----------------------------------------------------------------
// es_hip_matvec_multi_dev's job tables and pre-pass workspace, for callers that cannot allocate, live in this file-scope
// device array instead of a stream-ordered allocation: each device the library runs on holds its own copy until the
// process ends. Host code never passes the array's name (a host-side stand-in) to a kernel or a copy: it uses the device
// address hipGetSymbolAddress returns, looked up once per device with that device current.
constexpr size_t NOALLOC_SCRATCH = (size_t)ES_HIP_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH];

static std::mutex g_scratch_mu;
static std::vector<uint8_t *> g_scratch_dev;   // per device id: scratch's device address there (null: not looked up yet)

static int scratch_address(uint8_t **out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if ((size_t)dev >= g_scratch_dev.size()) g_scratch_dev.resize(dev + 1, nullptr);
    if (!g_scratch_dev[dev]) {
        void *p = nullptr;
        if ((e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))) != hipSuccess) return hip_fail(e, "hipGetSymbolAddress (scratch)");
        g_scratch_dev[dev] = static_cast<uint8_t *>(p);
    }
    *out = g_scratch_dev[dev];
    return ES_HIP_OK;
}

int es_hip_matvec_multi_dev_noalloc(uint32_t type, const void *W, int cols, int r0, int r1, const void *act, size_t astride,
                                    int na, float *y, size_t ystride, void *stream) {
    if (int rc = need_device()) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    // Not for graph capture: the job tables are copied from host memory that is gone when the call returns, and every
    // replay would share the one scratch array.
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone)
        return fail(ES_HIP_EINVAL, "es_hip_matvec_multi_dev_noalloc on a capturing stream: its job tables are copied from host "
                                   "memory at the call, so it cannot be recorded into a graph");
    std::vector<Req> reqs{{type, W, act, y, nullptr, nullptr, r0, r1, cols, na, astride, ystride}};
    Batch bt;
    if (int rc = plan_batch(reqs, bt)) return rc;
    if (bt.mm.empty() && bt.mqg.empty() && bt.mbg.empty() && bt.mkg.empty() && bt.pkg.empty())
        return bt.mv.empty() ? ES_HIP_OK : launch_single(bt.mv[0], s);
    const size_t ws_at = align256(bt.table_bytes), need = ws_at + bt.ws_bytes;
    if (need > NOALLOC_SCRATCH)
        return fail(ES_HIP_EINVAL, "this product needs %zu bytes of job tables and workspace, more than the %zu bytes of the "
                                   "no-allocation scratch (use es_hip_matvec_multi_dev)", need, NOALLOC_SCRATCH);
    uint8_t *dev = nullptr;
    if (int rc = scratch_address(&dev)) return rc;
    bind(bt, dev + ws_at);
    // Every pre-pass writes all of its padded planes (zeros past na), so nothing in the scratch needs clearing; the
    // tables are copied from pageable memory, which the copy has consumed when it returns.
    const std::vector<uint8_t> img = table_image(bt);
    hipError_t e;
    if (!img.empty() && (e = hipMemcpyAsync(dev, img.data(), img.size(), hipMemcpyHostToDevice, s)) != hipSuccess)
        return hip_fail(e, "job table upload");
    return launch_batch(bt, dev, g_order.load(), s);
}

int es_hip_matvec_dev(uint32_t type, const void *W, int cols, int r0, int r1, const void *act, float *y, void *stream) {
    return es_hip_matvec_multi_dev(type, W, cols, r0, r1, act, 0, 1, y, 0, stream);
}

int es_hip_block_ints_dev(uint32_t type, const void *W, int cols, int rows, const void *act, int32_t *dots, int32_t *aux,
                          void *stream) {
    if (int rc = need_device()) return rc;
    if (!dots || !aux) return fail(ES_HIP_EINVAL, "null dots/aux");
    void *ytmp = nullptr;
    std::lock_guard<std::mutex> lk(g_call_mu);
    if (int rc = g_ytmp.get((size_t)std::max(rows, 1) * sizeof(float), &ytmp)) return rc;
    std::vector<Req> reqs{{type, W, act, static_cast<float *>(ytmp), dots, aux, 0, rows, cols, 1, 0, 0}};
    std::vector<Group> groups;
    if (int rc = plan_groups(reqs, groups)) return rc;
    if (groups.empty()) return ES_HIP_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (int rc = launch_single(groups[0], s)) return rc;
    hipError_t e = hipStreamSynchronize(s);
    return e == hipSuccess ? ES_HIP_OK : hip_fail(e, "hipStreamSynchronize");
}

static void to_reqs(const es_hip_job *jobs, int njobs, std::vector<Req> &reqs) {
    reqs.clear();
    for (int i = 0; i < njobs; i++) {
        const es_hip_job &j = jobs[i];
        reqs.push_back({j.type, j.W, j.act, j.y, nullptr, nullptr, 0, j.rows, j.cols, j.nb, j.astride, j.ystride});
    }
}

int es_hip_run_jobs(const es_hip_job *jobs, int njobs, void *stream) {
    if (int rc = need_device()) return rc;
    if (njobs < 0 || (njobs > 0 && !jobs)) return fail(ES_HIP_EINVAL, "bad job list");
    std::vector<Req> reqs;
    to_reqs(jobs, njobs, reqs);
    std::lock_guard<std::mutex> lk(g_call_mu);
    return run_sync(reqs, static_cast<hipStream_t>(stream));
}

}  // extern "C"

struct es_hip_plan {
    Batch bt;
    uint8_t *dev = nullptr;   // job tables, then the pre-pass workspace
    int order;
    std::vector<es_hip_plan *> more;   // the later phases of long rows' column pieces, run after this one in order
    float *lanes = nullptr;            // their lane chains
};

static es_hip_plan *plan_one(const std::vector<Req> &reqs, int order) {
    auto *p = new es_hip_plan();
    p->order = order;
    if (plan_batch(reqs, p->bt)) { delete p; return nullptr; }
    const size_t ws_at = align256(p->bt.table_bytes);
    hipError_t e = hipMalloc(&p->dev, std::max<size_t>(ws_at + p->bt.ws_bytes, 256));
    if (e == hipSuccess) {
        bind(p->bt, p->dev + ws_at);
        const std::vector<uint8_t> img = table_image(p->bt);
        if (!img.empty()) e = hipMemcpy(p->dev, img.data(), img.size(), hipMemcpyHostToDevice);
    }
    if (e != hipSuccess) {
        hip_fail(e, "plan tables");
        es_hip_plan_destroy(p);
        return nullptr;
    }
    return p;
}

extern "C" {

es_hip_plan *es_hip_plan_create(const es_hip_job *jobs, int njobs) {
    if (need_device()) return nullptr;
    if (njobs < 0 || (njobs > 0 && !jobs)) { fail(ES_HIP_EINVAL, "bad job list"); return nullptr; }
    std::vector<Req> reqs;
    to_reqs(jobs, njobs, reqs);
    const int order = g_order.load();
    if (!has_long(reqs)) return plan_one(reqs, order);
    // rows past ES_HIP_MAX_COLS_*: one kept batch per phase of column pieces, the lane chains in the plan's own memory
    size_t nlanes = 0;
    if (count_lanes(reqs, order, nlanes)) return nullptr;
    float *lanes = nullptr;
    if (nlanes) {
        hipError_t e = hipMalloc(reinterpret_cast<void **>(&lanes), nlanes * sizeof(float));
        if (e != hipSuccess) { hip_fail(e, "hipMalloc (lane chains of long rows)"); return nullptr; }
    }
    std::vector<std::vector<Req>> phases;
    cut_pieces(reqs, order, lanes, phases);
    es_hip_plan *p = plan_one(phases[0], order);
    if (!p) { if (lanes) (void)hipFree(lanes); return nullptr; }
    p->lanes = lanes;
    for (size_t i = 1; i < phases.size(); i++) {
        es_hip_plan *m = plan_one(phases[i], order);
        if (!m) { es_hip_plan_destroy(p); return nullptr; }
        p->more.push_back(m);
    }
    return p;
}

int es_hip_plan_run(es_hip_plan *p, void *stream) {
    if (!p) return fail(ES_HIP_EINVAL, "null plan");
    int rc = launch_batch(p->bt, p->dev, p->order, static_cast<hipStream_t>(stream));
    for (es_hip_plan *m : p->more)
        if (!rc) rc = launch_batch(m->bt, m->dev, m->order, static_cast<hipStream_t>(stream));
    return rc;
}

void es_hip_plan_destroy(es_hip_plan *p) {
    if (!p) return;
    for (es_hip_plan *m : p->more) es_hip_plan_destroy(m);
    if (p->lanes) (void)hipFree(p->lanes);
    if (p->dev) (void)hipFree(p->dev);
    delete p;
}

int es_hip_set_mfma_min_batch(int n) { g_cfg_gen.fetch_add(1); return g_mm_min.exchange(n); }
int es_hip_set_mfma_tile(int bm, int bn, int waves) {
    g_cfg_gen.fetch_add(1);
    if (bm == 0 && bn == 0 && waves == 0) {
        g_mm_tile.store(0);
        return ES_HIP_OK;
    }
    if (!esq::mm_tile_ok(bm, bn, waves) || bn < 64) return fail(ES_HIP_EINVAL, "no %d x %d tile with %d waves", bm, bn, waves);
    g_mm_tile.store(bm | bn << 10 | waves << 20);
    return ES_HIP_OK;
}
int es_hip_set_small_batch_min(int n) { g_cfg_gen.fetch_add(1); return g_mq_min.exchange(n); }
int es_hip_set_batched32_min(int n) { g_cfg_gen.fetch_add(1); return g_mb_min.exchange(n); }
int es_hip_set_batched32_mfma_min(int n) { g_cfg_gen.fetch_add(1); return g_mbm_min.exchange(n); }
int es_hip_set_q6k_mfma_min_batch(int n) { g_cfg_gen.fetch_add(1); return g_mm6_min.exchange(n); }
int es_hip_set_q2k_mfma_min_batch(int n) { g_cfg_gen.fetch_add(1); return g_mm2_min.exchange(n); }
int es_hip_set_direct_mfma_min_batch(int n) { g_cfg_gen.fetch_add(1); return g_mk_min.exchange(n); }
int es_hip_set_direct_mfma_min_tiles(int n) { g_cfg_gen.fetch_add(1); return g_mk_min_tiles.exchange(n); }
int es_hip_set_q5k_mfma_min_batch(int n) { g_cfg_gen.fetch_add(1); return g_mk5_min.exchange(n); }
int es_hip_set_q3k_mfma_min_batch(int n) { g_cfg_gen.fetch_add(1); return g_mk3_min.exchange(n); }
int es_hip_set_direct_persistent(int on) {
    g_cfg_gen.fetch_add(1);
    return g_pk_on.exchange(on == 2 || on == 3 ? on : on ? 1 : 0);
}
int es_hip_set_q2k_expert_max_batch(int n) { g_cfg_gen.fetch_add(1); return g_mx_max.exchange(n); }
int es_hip_set_moe_gated(int on) { g_cfg_gen.fetch_add(1); return g_moe_gated.exchange(on != 0 ? 1 : 0); }
int es_hip_set_batched32_direct(int on) { g_cfg_gen.fetch_add(1); return g_mbx_on.exchange(on ? 1 : 0); }
int es_hip_set_q6k_persistent(int on) { g_cfg_gen.fetch_add(1); return esq::mm6_set_persistent(on); }
int es_hip_set_direct_mfma_tok64(int on) { g_cfg_gen.fetch_add(1); return g_mk_tok64.exchange(on ? 1 : 0); }

double es_hip_plan_time_ms(es_hip_plan *p, int warmup, int iters, void *stream) {
    if (!p || iters <= 0) { fail(ES_HIP_EINVAL, "bad plan or iteration count"); return -1.0; }
    hipStream_t s = static_cast<hipStream_t>(stream);
    for (int i = 0; i < warmup; i++)
        if (es_hip_plan_run(p, stream)) return -1.0;
    hipEvent_t a, b;
    if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) { fail(ES_HIP_ERUNTIME, "hipEventCreate"); return -1.0; }
    (void)hipEventRecord(a, s);
    for (int i = 0; i < iters; i++)
        if (es_hip_plan_run(p, stream)) return -1.0;
    (void)hipEventRecord(b, s);
    (void)hipEventSynchronize(b);
    float ms = 0.0f;
    (void)hipEventElapsedTime(&ms, a, b);
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    return (double)ms / iters;
}

// ---- weight registry and host-memory drop-ins ---------------------------------------------------------------------
int es_hip_register(const void *host, size_t bytes) {
    if (int rc = need_device()) return rc;
    if (!host || !bytes) return fail(ES_HIP_EINVAL, "empty registration");
    es_hip_unregister(host);
    void *d = nullptr;
    hipError_t e = hipMalloc(&d, bytes);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc (register)");
    e = hipMemcpy(d, host, bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) { (void)hipFree(d); return hip_fail(e, "hipMemcpy (register)"); }
    std::lock_guard<std::mutex> lk(g_reg_mu);
    g_reg[reinterpret_cast<uintptr_t>(host)] = {bytes, d};
    return ES_HIP_OK;
}

int es_hip_update(const void *host) {
    if (int rc = need_device()) return rc;
    std::lock_guard<std::mutex> lk(g_reg_mu);
    auto it = g_reg.find(reinterpret_cast<uintptr_t>(host));
    if (it == g_reg.end()) return fail(ES_HIP_EINVAL, "not registered");
    hipError_t e = hipMemcpy(it->second.dev, host, it->second.bytes, hipMemcpyHostToDevice);
    return e == hipSuccess ? ES_HIP_OK : hip_fail(e, "hipMemcpy (update)");
}

int es_hip_unregister(const void *host) {
    std::lock_guard<std::mutex> lk(g_reg_mu);
    auto it = g_reg.find(reinterpret_cast<uintptr_t>(host));
    if (it == g_reg.end()) return ES_HIP_EINVAL;
    (void)hipFree(it->second.dev);
    g_reg.erase(it);
    return ES_HIP_OK;
}

// The activation blocks the format takes (Q8_0 for the 32-element formats, Q8_K for the K-quants), or NULL when the
// activation was prepared without them: es_act_prepare without a Q8_K buffer, with its Q8_0 arena exhausted, or under
// ES_FLOAT_ACT (src/es_quant.c:499-512). Such an activation takes the reference's float path (src/es_quant.c:1941-1944).
static const void *act_blocks(const FmtInfo &f, const es_hip_act &a) {
    return f.be == 32 ? static_cast<const void *>(a.q80) : static_cast<const void *>(a.q8);
}

// Splits a host activation list into those with blocks (integer path) and those without (float path, which needs x).
static int split_acts(const FmtInfo &f, const es_hip_act *a, int na, std::vector<int> &qi, std::vector<int> &qf, int job) {
    qi.clear();
    qf.clear();
    for (int q = 0; q < na; q++) {
        if (act_blocks(f, a[q])) qi.push_back(q);
        else if (a[q].x) qf.push_back(q);
        else if (job < 0) return fail(ES_HIP_EINVAL, "activation %d has neither %s blocks nor floats", q, f.be == 32 ? "Q8_0" : "Q8_K");
        else return fail(ES_HIP_EINVAL, "job %d activation %d has neither %s blocks nor floats", job, q, f.be == 32 ? "Q8_0" : "Q8_K");
    }
    return ES_HIP_OK;
}

static int float_launch(uint32_t type, const void *dW, size_t rb, int rows, int cols, const float *x, int na, float *y,
                        hipStream_t s) {
    if (reinterpret_cast<uintptr_t>(dW) & 1) return fail(ES_HIP_EINVAL, "W must be 2-byte aligned");
    hipError_t e = esq::fdot_launch(type, dW, rb, 0, rows, cols, x, (size_t)cols, na, y, (size_t)rows, s);
    return e == hipSuccess ? ES_HIP_OK : hip_fail(e, "float-path launch");
}

static int host_multi(uint32_t type, const void *W, int cols, int r0, int r1, const es_hip_act *a, int na, float *y,
                      size_t ystride, int order = -1) {
    g_err.clear();   // the void drop-ins report failure only through es_hip_last_error()
    if (int rc = need_device()) return rc;
    FmtInfo f;
    if (!fmt_info(type, f)) return fail(ES_HIP_EINVAL, "type %u is not computed by this library", type);
    if (cols <= 0 || cols % f.be || r0 < 0 || r1 < r0 || na < 0) return fail(ES_HIP_EINVAL, "bad shape");
    if (r1 == r0 || na == 0) return ES_HIP_OK;
    if (!W || !a || !y) return fail(ES_HIP_EINVAL, "null pointer");
    const int nbk = cols / f.be;
    const size_t rb = (size_t)nbk * f.bb, ab = (size_t)nbk * f.ab;
    const int n = r1 - r0;
    std::vector<int> qi, qf;   // activations with blocks, then those on the float path; outputs in that order
    if (int rc = split_acts(f, a, na, qi, qf, -1)) return rc;
    std::lock_guard<std::mutex> lk(g_call_mu);
    if (int rc = settle()) return rc;
    const uint8_t *wsub = static_cast<const uint8_t *>(W) + rb * r0;
    const void *dW = reg_lookup(wsub, rb * n);
    void *wt = nullptr, *at = nullptr, *yt = nullptr;
    hipError_t e;
    if (!dW) {   // not resident: upload the rows for this call
        if (int rc = g_wtmp.get(rb * n, &wt)) return rc;
        if ((e = hipMemcpy(wt, wsub, rb * n, hipMemcpyHostToDevice)) != hipSuccess) return hip_fail(e, "weight upload");
        dW = wt;
    }
    const size_t ibytes = align256(ab * qi.size()), xbytes = sizeof(float) * cols * qf.size();
    void *hin = nullptr, *hout = nullptr;
    if (int rc = g_atmp.get(ibytes + xbytes, &at)) return rc;
    if (int rc = g_hin.get(ibytes + xbytes, &hin)) return rc;
    std::vector<HCopy> cp;
    uint8_t *pack = static_cast<uint8_t *>(hin);
    for (size_t k = 0; k < qi.size(); k++) cp.push_back({pack + ab * k, act_blocks(f, a[qi[k]]), ab});
    for (size_t k = 0; k < qf.size(); k++) cp.push_back({pack + ibytes + sizeof(float) * cols * k, a[qf[k]].x, sizeof(float) * cols});
    host_copies(cp);
    g_table_pending = true;
    if ((e = hipMemcpyAsync(at, hin, ibytes + xbytes, hipMemcpyHostToDevice, nullptr)) != hipSuccess) return hip_fail(e, "activation upload");
    if (int rc = g_ytmp.get(sizeof(float) * n * na, &yt)) return rc;
    float *yd = static_cast<float *>(yt);
    if (!qf.empty())
        if (int rc = float_launch(type, dW, rb, n, cols, reinterpret_cast<const float *>(static_cast<uint8_t *>(at) + ibytes),
                                  (int)qf.size(), yd + (size_t)n * qi.size(), nullptr))
            return rc;
    if (!qi.empty()) {
        std::vector<Req> reqs{{type, dW, at, yd, nullptr, nullptr, 0, n, cols, (int)qi.size(), ab, (size_t)n}};
        if (int rc = run_launch(reqs, nullptr, order)) return rc;
    }
    if (int rc = g_hout.get(sizeof(float) * n * na, &hout)) return rc;
    if ((e = hipMemcpyAsync(hout, yt, sizeof(float) * n * na, hipMemcpyDeviceToHost, nullptr)) != hipSuccess)
        return hip_fail(e, "output download");
    if (int rc = finish(nullptr)) return rc;
    qi.insert(qi.end(), qf.begin(), qf.end());
    const float *out = static_cast<const float *>(hout);
    cp.clear();
    for (int k = 0; k < na; k++) cp.push_back({y + ystride * qi[k] + r0, out + (size_t)n * k, sizeof(float) * n});
    host_copies(cp);
    return ES_HIP_OK;
}

int es_hip_run_jobs_host(const es_hip_host_job *jobs, int njobs) {
    if (int rc = need_device()) return rc;
    if (njobs < 0 || (njobs > 0 && !jobs)) return fail(ES_HIP_EINVAL, "bad job list");
    // sizes of the staged activations (blocks, then the float-path activations' floats), outputs and unregistered weights
    struct Stage { size_t aoff, xoff, yoff, woff; const void *dW; size_t ab, rb; std::vector<int> qi, qf; };
    std::vector<Stage> st(njobs);
    size_t abytes = 0, ybytes = 0, wbytes = 0;
    for (int i = 0; i < njobs; i++) {
        const es_hip_host_job &j = jobs[i];
        FmtInfo f;
        if (!fmt_info(j.type, f)) return fail(ES_HIP_EINVAL, "job %d: type %u is not computed by this library", i, j.type);
        if (j.cols <= 0 || j.cols % f.be || j.rows < 0 || j.nb < 0) return fail(ES_HIP_EINVAL, "job %d: bad shape", i);
        if (j.rows == 0 || j.nb == 0) continue;
        if (!j.w || !j.a || !j.y) return fail(ES_HIP_EINVAL, "job %d: null pointer", i);
        const int nbk = j.cols / f.be;
        st[i].ab = (size_t)nbk * f.ab;
        st[i].rb = (size_t)nbk * f.bb;
        if (int rc = split_acts(f, j.a, j.nb, st[i].qi, st[i].qf, i)) return rc;
        st[i].aoff = abytes;
        abytes += align256(st[i].ab * st[i].qi.size());
        st[i].xoff = abytes;
        abytes += align256(sizeof(float) * j.cols * st[i].qf.size());
        st[i].yoff = ybytes;
        ybytes += align256((size_t)j.rows * j.nb * sizeof(float));
        st[i].dW = reg_lookup(j.w, st[i].rb * j.rows);
        if (!st[i].dW) { st[i].woff = wbytes; wbytes += align256(st[i].rb * j.rows); }
    }
    std::lock_guard<std::mutex> lk(g_call_mu);
    if (int rc = settle()) return rc;
    void *at = nullptr, *yt = nullptr, *wt = nullptr;
    if (abytes)
        if (int rc = g_atmp.get(abytes, &at)) return rc;
    if (ybytes)
        if (int rc = g_ytmp.get(ybytes, &yt)) return rc;
    if (wbytes)
        if (int rc = g_wtmp.get(wbytes, &wt)) return rc;
    void *hin = nullptr, *hout = nullptr;
    if (abytes)
        if (int rc = g_hin.get(abytes, &hin)) return rc;
    if (ybytes)
        if (int rc = g_hout.get(ybytes, &hout)) return rc;
    uint8_t *pack = static_cast<uint8_t *>(hin);
    std::vector<HCopy> cp;
    std::vector<Req> reqs;
    hipError_t e;
    for (int i = 0; i < njobs; i++) {
        const es_hip_host_job &j = jobs[i];
        if (j.rows == 0 || j.nb == 0) continue;
        FmtInfo f;
        fmt_info(j.type, f);
        const Stage &g = st[i];
        for (size_t k = 0; k < g.qi.size(); k++) cp.push_back({pack + g.aoff + g.ab * k, act_blocks(f, j.a[g.qi[k]]), g.ab});
        for (size_t k = 0; k < g.qf.size(); k++)
            cp.push_back({pack + g.xoff + sizeof(float) * j.cols * k, j.a[g.qf[k]].x, sizeof(float) * j.cols});
        const void *dW = g.dW;
        if (!dW) {
            dW = static_cast<uint8_t *>(wt) + g.woff;
            if ((e = hipMemcpy(const_cast<void *>(dW), j.w, g.rb * j.rows, hipMemcpyHostToDevice)) != hipSuccess)
                return hip_fail(e, "weight upload");
        }
        float *yd = reinterpret_cast<float *>(static_cast<uint8_t *>(yt) + g.yoff);
        if (!g.qi.empty())
            reqs.push_back({j.type, dW, static_cast<uint8_t *>(at) + g.aoff, yd, nullptr, nullptr, 0, j.rows, j.cols,
                            (int)g.qi.size(), g.ab, (size_t)j.rows});
    }
    host_copies(cp);
    g_table_pending = true;
    if (abytes && (e = hipMemcpyAsync(at, hin, abytes, hipMemcpyHostToDevice, nullptr)) != hipSuccess)
        return hip_fail(e, "activation upload");
    for (int i = 0; i < njobs; i++) {   // the float-path activations, stream-ordered before the batch's launches
        const es_hip_host_job &j = jobs[i];
        const Stage &g = st[i];
        if (j.rows == 0 || j.nb == 0 || g.qf.empty()) continue;
        const void *dW = g.dW ? g.dW : static_cast<uint8_t *>(wt) + g.woff;
        float *yd = reinterpret_cast<float *>(static_cast<uint8_t *>(yt) + g.yoff) + (size_t)j.rows * g.qi.size();
        if (int rc = float_launch(j.type, dW, g.rb, j.rows, j.cols,
                                  reinterpret_cast<const float *>(static_cast<uint8_t *>(at) + g.xoff), (int)g.qf.size(), yd,
                                  nullptr))
            return rc;
    }
    if (int rc = run_launch(reqs, nullptr, -1)) return rc;
    if (ybytes && (e = hipMemcpyAsync(hout, yt, ybytes, hipMemcpyDeviceToHost, nullptr)) != hipSuccess)
        return hip_fail(e, "output download");
    if (int rc = finish(nullptr)) return rc;
    cp.clear();
    for (int i = 0; i < njobs; i++) {
        const es_hip_host_job &j = jobs[i];
        if (j.rows == 0 || j.nb == 0) continue;
        const float *src = reinterpret_cast<const float *>(static_cast<const uint8_t *>(hout) + st[i].yoff);
        int k = 0;
        for (int q : st[i].qi) cp.push_back({j.y + j.ys * q, src + (size_t)j.rows * k++, sizeof(float) * j.rows});
        for (int q : st[i].qf) cp.push_back({j.y + j.ys * q, src + (size_t)j.rows * k++, sizeof(float) * j.rows});
    }
    host_copies(cp);
    return ES_HIP_OK;
}

void es_hip_matvec(uint32_t type, const void *W, int cols, int r0, int r1, const es_hip_act *a, float *y, float *scratch) {
    (void)scratch;
    host_multi(type, W, cols, r0, r1, a, 1, y, 0);
}

void es_hip_matvec_multi(uint32_t type, const void *W, int cols, int r0, int r1, const es_hip_act *a, int na, float *y,
                         size_t ystride, float *scratch) {
    (void)scratch;
    host_multi(type, W, cols, r0, r1, a, na, y, ystride);
}

// es_matvec_q2_K (src/es_q2k.c:223-229) runs the portable dot (or, forced, es_dot_q2_K_q8_K_ref: the same float order,
// src/es_q2k.c:127-148, 160-190) in every build: per block sumf += dall * isum - dmin * summs, nothing fused
static std::atomic<int> g_q2k_scalar{0};

void es_hip_matvec_q2_K(const void *W, int cols, int r0, int r1, const void *xq, float *y) {
    es_hip_act a{nullptr, static_cast<es_hip_block_q8_K *>(const_cast<void *>(xq)), nullptr, cols};
    host_multi(ES_HIP_Q2_K, W, cols, r0, r1, &a, 1, y, 0, ES_HIP_ORDER_X86_STRICT);
}

const char *es_hip_q2k_kernel_name(void) { return g_q2k_scalar.load() ? "hip-gfx950 (scalar order)" : "hip-gfx950"; }

void es_hip_q2k_force_scalar(int on) { g_q2k_scalar.store(on ? 1 : 0); }

}  // extern "C"

// ---- MoE expert FFN ---------------------------------------------------------------------------------------------------
struct es_hip_moe_plan {
    Batch gu, dn;                // gate/up products, down products
    uint8_t *bufs = nullptr;     // gather table, combine tables, gate|up outputs, requantized h, expert outputs
    uint8_t *tabs = nullptr;     // job tables and pre-pass workspaces of both batches
    size_t gu_tab = 0, dn_tab = 0;
    int order = 0;
    int rows = 0, ff = 0, n = 0, ntok = 0, kmax = 0;
    bool h_q8k = true;
    bool gated = false;          // gate/up on the gated expert kernel: h written as Q8_K blocks, no SwiGLU launch
    uint64_t hstride = 0, ostride = 0;
    float *bgu = nullptr, *bye = nullptr, *out = nullptr, *w = nullptr;
    uint8_t *ha = nullptr;
    int *rowof = nullptr, *kk = nullptr;
};

namespace {

// moe_n's grouping (src/es_engine.c:871-888): distinct experts in order of first use, each pair's row grouped by expert
void moe_group(int ntok, const int *k, const int *sel, int kmax, std::vector<int> &uex, std::vector<int> &cnt,
               std::vector<int> &start, std::vector<int> &rowof, std::vector<int> &tok_of) {
    uex.clear();
    cnt.clear();
    std::vector<int> slot(ntok * (size_t)kmax, -1);
    for (int t = 0; t < ntok; t++)
        for (int j = 0; j < k[t]; j++) {
            const int e = sel[t * kmax + j];
            size_t u = 0;
            while (u < uex.size() && uex[u] != e) u++;
            if (u == uex.size()) { uex.push_back(e); cnt.push_back(0); }
            cnt[u]++;
            slot[t * (size_t)kmax + j] = (int)u;
        }
    start.assign(uex.size(), 0);
    for (size_t u = 0, r = 0; u < uex.size(); u++) { start[u] = (int)r; r += cnt[u]; }
    std::vector<int> fill(uex.size(), 0);
    rowof.assign(ntok * (size_t)kmax, 0);
    tok_of.clear();
    int total = 0;
    for (int c : cnt) total += c;
    tok_of.assign(total, 0);
    for (int t = 0; t < ntok; t++)
        for (int j = 0; j < k[t]; j++) {
            const int u = slot[t * (size_t)kmax + j], r = start[u] + fill[u]++;
            rowof[t * (size_t)kmax + j] = r;
            tok_of[r] = t;
        }
}

int moe_build(es_hip_moe_plan *p, const es_hip_moe *m, int N, const int *k, const int *sel, const float *w, int kmax,
              const void *x, size_t xstride, float *out, size_t ostride) {
    if (!m) return fail(ES_HIP_EINVAL, "null expert set");
    FmtInfo fg, fu, fd;
    if (!fmt_info(m->gate_type, fg) || !fmt_info(m->up_type, fu) || !fmt_info(m->down_type, fd))
        return fail(ES_HIP_EINVAL, "an expert type is not computed by this library");
    if (fg.be != fu.be) return fail(ES_HIP_EINVAL, "gate and up take different activation blocks");
    if (m->n <= 0 || m->ff <= 0 || m->n % fg.be || m->ff % fd.be) return fail(ES_HIP_EINVAL, "bad widths n %d, ff %d", m->n, m->ff);
    if (m->n_exp <= 0 || !m->gate || !m->up || !m->down) return fail(ES_HIP_EINVAL, "bad expert table");
    if (N < 0 || kmax <= 0 || (N > 0 && (!k || !sel || !w || !x || !out))) return fail(ES_HIP_EINVAL, "bad routing or buffers");
    if (ostride == 0) ostride = (size_t)m->n;
    if (N > 1 && ostride < (size_t)m->n) return fail(ES_HIP_EINVAL, "ostride %zu < n %d", ostride, m->n);
    for (int t = 0; t < N; t++) {
        if (k[t] < 0 || k[t] > kmax) return fail(ES_HIP_EINVAL, "token %d: k %d outside [0, %d]", t, k[t], kmax);
        for (int j = 0; j < k[t]; j++) {
            const int e = sel[t * kmax + j];
            if (e < 0 || e >= m->n_exp) return fail(ES_HIP_EINVAL, "token %d: expert %d outside [0, %d)", t, e, m->n_exp);
            if (!m->gate[e] || !m->up[e] || !m->down[e]) return fail(ES_HIP_EINVAL, "expert %d is routed but has no weights", e);
        }
    }
    std::vector<int> uex, cnt, start, rowof, tok_of;
    moe_group(N, k, sel, kmax, uex, cnt, start, rowof, tok_of);
    const int R = (int)tok_of.size(), n = m->n, ff = m->ff;
    p->order = g_order.load();
    p->rows = R;
    p->ff = ff;
    p->n = n;
    p->ntok = N;
    p->kmax = kmax;
    p->h_q8k = fd.be == 256;
    p->hstride = (uint64_t)(ff / fd.be) * fd.ab;
    p->ostride = ostride;
    p->out = out;
    // fixed buffers
    size_t off = 0;
    const size_t o_arow = off;  off += align256(sizeof(int) * std::max(R, 1));
    const size_t o_rowof = off; off += align256(sizeof(int) * std::max<size_t>(rowof.size(), 1));
    const size_t o_w = off;     off += align256(sizeof(float) * std::max<size_t>(rowof.size(), 1));
    const size_t o_k = off;     off += align256(sizeof(int) * std::max(N, 1));
    const size_t o_gu = off;    off += align256(sizeof(float) * 2 * ff * (size_t)std::max(R, 1));
    const size_t o_ha = off;    off += align256(p->hstride * std::max(R, 1));
    const size_t o_ye = off;    off += align256(sizeof(float) * n * (size_t)std::max(R, 1));
    hipError_t e = hipMalloc(&p->bufs, off);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc (MoE buffers)");
    int *arow = reinterpret_cast<int *>(p->bufs + o_arow);
    p->rowof = reinterpret_cast<int *>(p->bufs + o_rowof);
    p->w = reinterpret_cast<float *>(p->bufs + o_w);
    p->kk = reinterpret_cast<int *>(p->bufs + o_k);
    p->bgu = reinterpret_cast<float *>(p->bufs + o_gu);
    p->ha = p->bufs + o_ha;
    p->bye = reinterpret_cast<float *>(p->bufs + o_ye);
    std::vector<float> wv(rowof.size(), 0.0f);
    for (int t = 0; t < N; t++)
        for (int j = 0; j < k[t]; j++) wv[t * (size_t)kmax + j] = w[t * kmax + j];
    std::vector<int> kv(k, k + N);
    if ((R && (e = hipMemcpy(arow, tok_of.data(), sizeof(int) * R, hipMemcpyHostToDevice)) != hipSuccess) ||
        (N && (e = hipMemcpy(p->rowof, rowof.data(), sizeof(int) * rowof.size(), hipMemcpyHostToDevice)) != hipSuccess) ||
        (N && (e = hipMemcpy(p->w, wv.data(), sizeof(float) * wv.size(), hipMemcpyHostToDevice)) != hipSuccess) ||
        (N && (e = hipMemcpy(p->kk, kv.data(), sizeof(int) * N, hipMemcpyHostToDevice)) != hipSuccess))
        return hip_fail(e, "MoE table upload");
    // the two grouped products
    const uint64_t xs = xstride ? xstride : (uint64_t)(n / fg.be) * fg.ab;
    std::vector<Req> gu, dn;
    // experts with the most tokens first: their workgroups run longest, so they start first and the launch ends evenly
    std::vector<int> ord(uex.size());
    for (size_t u = 0; u < ord.size(); u++) ord[u] = (int)u;
    std::stable_sort(ord.begin(), ord.end(), [&](int a, int b) { return cnt[a] > cnt[b]; });
    // Q2_K gate and up with a K-quant down: one gated product per expert when every expert's fits the gated kernel
    auto gated_req = [&](int ex, int s0, int c) {
        return Req{m->gate_type, m->gate[ex], x, reinterpret_cast<float *>(p->ha + (size_t)s0 * p->hstride), nullptr, nullptr,
                   0, ff, n, c, xs, (size_t)p->hstride, arow + s0, N, m->up[ex]};
    };
    p->gated = g_moe_gated.load() && m->gate_type == ES_HIP_Q2_K && m->up_type == ES_HIP_Q2_K && p->h_q8k;
    for (size_t u = 0; u < uex.size() && p->gated; u++) p->gated = mx_eligible(gated_req(uex[u], start[u], cnt[u]));
    for (int u : ord) {
        const int ex = uex[u], s0 = start[u], c = cnt[u];
        float *y = p->bgu + (size_t)s0 * 2 * ff;
        if (p->gated) {
            gu.push_back(gated_req(ex, s0, c));
        } else {
            gu.push_back({m->gate_type, m->gate[ex], x, y, nullptr, nullptr, 0, ff, n, c, xs, (size_t)2 * ff, arow + s0, N});
            gu.push_back({m->up_type, m->up[ex], x, y + ff, nullptr, nullptr, 0, ff, n, c, xs, (size_t)2 * ff, arow + s0, N});
        }
        dn.push_back({m->down_type, m->down[ex], p->ha + (size_t)s0 * p->hstride, p->bye + (size_t)s0 * n, nullptr, nullptr, 0, n,
                      ff, c, p->hstride, (size_t)n, nullptr});
    }
    if (int rc = plan_batch(gu, p->gu)) return rc;
    if (int rc = plan_batch(dn, p->dn)) return rc;
    const size_t gu_ws = align256(p->gu.table_bytes), dn_tab = align256(gu_ws + p->gu.ws_bytes),
                 dn_ws = align256(dn_tab + p->dn.table_bytes), total = dn_ws + p->dn.ws_bytes;
    if ((e = hipMalloc(&p->tabs, std::max<size_t>(total, 256))) != hipSuccess) return hip_fail(e, "hipMalloc (MoE tables)");
    p->gu_tab = 0;
    p->dn_tab = dn_tab;
    bind(p->gu, p->tabs + gu_ws);
    bind(p->dn, p->tabs + dn_ws);
    const std::vector<uint8_t> gi = table_image(p->gu), di = table_image(p->dn);
    if ((!gi.empty() && (e = hipMemcpy(p->tabs, gi.data(), gi.size(), hipMemcpyHostToDevice)) != hipSuccess) ||
        (!di.empty() && (e = hipMemcpy(p->tabs + dn_tab, di.data(), di.size(), hipMemcpyHostToDevice)) != hipSuccess))
        return hip_fail(e, "MoE job tables");
    return ES_HIP_OK;
}

int moe_run(const es_hip_moe_plan *p, hipStream_t s) {
    if (int rc = launch_batch(p->gu, p->tabs + p->gu_tab, p->order, s)) return rc;
    hipError_t e = p->gated ? hipSuccess : esq::moe_swiglu_launch(p->bgu, p->rows, p->ff, p->h_q8k, p->ha, p->hstride, s);
    if (e != hipSuccess) return hip_fail(e, "SwiGLU launch");
    if (int rc = launch_batch(p->dn, p->tabs + p->dn_tab, p->order, s)) return rc;
    e = esq::moe_combine_launch(p->bye, p->rowof, p->w, p->kk, p->kmax, p->ntok, p->n, p->out, p->ostride, s);
    return e == hipSuccess ? ES_HIP_OK : hip_fail(e, "combine launch");
}

}  // namespace

// error reporting and device discovery for the library's other host files (es_hip_host.h)
namespace esq {
int host_fail(int code, const char *msg) { return fail(code, "%s", msg); }
int host_hip_fail(hipError_t e, const char *what) { return hip_fail(e, what); }
int host_need_device() { return need_device(); }
}  // namespace esq

extern "C" {

es_hip_moe_plan *es_hip_moe_plan_create(const es_hip_moe *m, int N, const int *k, const int *sel, const float *w, int kmax,
                                        const void *x, size_t xstride, float *out, size_t ostride) {
    if (need_device()) return nullptr;
    auto *p = new es_hip_moe_plan();
    if (moe_build(p, m, N, k, sel, w, kmax, x, xstride, out, ostride)) {
        es_hip_moe_plan_destroy(p);
        return nullptr;
    }
    return p;
}

int es_hip_moe_plan_run(es_hip_moe_plan *p, void *stream) {
    if (!p) return fail(ES_HIP_EINVAL, "null plan");
    return moe_run(p, static_cast<hipStream_t>(stream));
}

void es_hip_moe_plan_destroy(es_hip_moe_plan *p) {
    if (!p) return;
    if (p->bufs) (void)hipFree(p->bufs);
    if (p->tabs) (void)hipFree(p->tabs);
    delete p;
}

double es_hip_step_time_ms(es_hip_plan *const *plans, int np, es_hip_moe_plan *const *moe, int nm, int warmup, int iters,
                           void *stream) {
    if (np < 0 || nm < 0 || iters <= 0 || (np && !plans) || (nm && !moe)) { fail(ES_HIP_EINVAL, "bad step"); return -1.0; }
    hipStream_t s = static_cast<hipStream_t>(stream);
    auto one = [&]() {
        for (int i = 0; i < np; i++)
            if (es_hip_plan_run(plans[i], stream)) return false;
        for (int i = 0; i < nm; i++)
            if (es_hip_moe_plan_run(moe[i], stream)) return false;
        return true;
    };
    for (int i = 0; i < warmup; i++)
        if (!one()) return -1.0;
    hipEvent_t a, b;
    if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) { fail(ES_HIP_ERUNTIME, "hipEventCreate"); return -1.0; }
    (void)hipEventRecord(a, s);
    for (int i = 0; i < iters; i++)
        if (!one()) return -1.0;
    (void)hipEventRecord(b, s);
    (void)hipEventSynchronize(b);
    float ms = 0.0f;
    (void)hipEventElapsedTime(&ms, a, b);
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    return (double)ms / iters;
}

int es_hip_moe_ffn(const es_hip_moe *m, int N, const int *k, const int *sel, const float *w, int kmax, const void *x,
                   size_t xstride, float *out, size_t ostride, void *stream) {
    if (int rc = need_device()) return rc;
    es_hip_moe_plan p;
    int rc = moe_build(&p, m, N, k, sel, w, kmax, x, xstride, out, ostride);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (!rc) rc = moe_run(&p, s);
    hipError_t e = hipStreamSynchronize(s);   // the plan's buffers are freed below
    if (!rc && e != hipSuccess) rc = hip_fail(e, "hipStreamSynchronize");
    if (p.bufs) (void)hipFree(p.bufs);
    if (p.tabs) (void)hipFree(p.tabs);
    return rc;
}

int es_hip_moe_ffn_logits(const es_hip_moe *m, int N, const float *logits, size_t lstride, int k, int norm_topk,
                          const void *x, size_t xstride, float *out, size_t ostride, int *sel_out, float *w_out,
                          void *stream) {
    if (int rc = need_device()) return rc;
    if (!m) return fail(ES_HIP_EINVAL, "null MoE description");
    if (N < 0 || k <= 0) return fail(ES_HIP_EINVAL, "bad token count %d or top-k %d", N, k);
    if (N == 0) return ES_HIP_OK;
    const size_t pairs = (size_t)N * k;
    void *buf = nullptr;
    hipError_t e = hipMalloc(&buf, pairs * (sizeof(int) + sizeof(float)));
    if (e != hipSuccess) return hip_fail(e, "hipMalloc (routing)");
    int *dsel = static_cast<int *>(buf);
    float *dw = reinterpret_cast<float *>(dsel + pairs);
    hipStream_t s = static_cast<hipStream_t>(stream);
    std::vector<int> sel(pairs), kk((size_t)N, k);
    std::vector<float> w(pairs);
    int rc = es_hip_route_softmax_dev(logits, lstride, N, m->n_exp, k, norm_topk, dsel, dw, k, stream);
    if (!rc && ((e = hipMemcpyAsync(sel.data(), dsel, pairs * sizeof(int), hipMemcpyDeviceToHost, s)) != hipSuccess ||
                (e = hipMemcpyAsync(w.data(), dw, pairs * sizeof(float), hipMemcpyDeviceToHost, s)) != hipSuccess ||
                (e = hipStreamSynchronize(s)) != hipSuccess))
        rc = hip_fail(e, "routing copy to the host");
    (void)hipFree(buf);
    if (rc) return rc;
    if (sel_out) std::memcpy(sel_out, sel.data(), pairs * sizeof(int));
    if (w_out) std::memcpy(w_out, w.data(), pairs * sizeof(float));
    return es_hip_moe_ffn(m, N, kk.data(), sel.data(), w.data(), k, x, xstride, out, ostride, stream);
}

}  // extern "C"

// ---- device-routed MoE context ----------------------------------------------------------------------------------------
// Buffers for up to max_tokens tokens and every table of the two launches, allocated once; a layer then runs in stream
// order with no allocation, no copy to or from the host and no wait: routing (optional), grouping and job tables on the
// device (moe_group_build), gate/up, SwiGLU + requantization, down, combine.
struct es_hip_moe_ctx {
    uint32_t gt, ut, dt;
    int n, ff, n_exp, max_tokens, k;
    uint8_t *buf = nullptr;
    int *sel = nullptr, *tok_of = nullptr, *rowof = nullptr, *kk = nullptr;
    float *w = nullptr, *wv = nullptr, *bgu = nullptr, *bye = nullptr;
    uint8_t *ha = nullptr;
    const uint8_t **dgate = nullptr, **dup = nullptr, **ddown = nullptr;
    void *gu_jobs = nullptr, *dn_jobs = nullptr;
    esq::PrepJob *gu_prep = nullptr, *dn_prep = nullptr;
    uint8_t *gu_ws = nullptr, *dn_ws = nullptr;
    uint64_t hstride = 0, gu_slot = 0, dn_slot = 0;   // gu_slot / dn_slot: plane workspace bytes
    const uint8_t *w_gate0 = nullptr, *w_down0 = nullptr;   // a valid weight pointer for empty jobs
    bool h_q8k = true;
    std::map<std::array<int, 6>, std::pair<MvLaunch, MvJob>> mv_cache;   // decode-kernel sizing by (type, rows, cols, ...)
};

namespace {

// na_pad and tile activations of a matrix-core product of about `na` activations (the planner's rule for one product)
bool moe_mm_family(uint32_t type, int cols, double expect, int &bn) {
    const Req q{type, nullptr, nullptr, nullptr, nullptr, nullptr, 0, 1, cols, std::max(1, (int)(expect + 0.5)), 0, 0};
    if (!mm_eligible(q)) return false;
    const int na = q.na;
    if (type == ES_HIP_Q2_K) bn = na <= 32 ? 32 : 64;
    else if (type == ES_HIP_Q6_K) bn = na <= 16 ? 16 : na <= 32 ? 32 : 64;
    else bn = na <= 16 ? 16 : na <= 32 ? 32 : na <= 64 ? 64 : 128;
    return esq::mm_tile_ok(128, bn, 8);
}

// the expert-sized kernel for a MoE product when plan_batch would pick it at the expected count per expert, with its
// 32-bit offsets in range: the act_rows activation rows within 4 GiB of the first, the outputs (R + MX_TOK activations
// past any expert's first) within 2 GiB
bool moe_mx_family(uint32_t type, int rows, int cols, double expect, int R, size_t act_rows, uint64_t astride,
                   uint64_t ystride) {
    const int na = std::max(1, (int)(expect + 0.5));
    return type == ES_HIP_Q2_K && na >= 2 && na <= g_mx_max.load() && cols / 256 <= esq::MX_NBK && rows > 0 &&
           act_rows * astride < ((size_t)1 << 32) - 65536 &&
           ((size_t)R + esq::MX_TOK) * ystride * sizeof(float) < ((size_t)1 << 31);
}

// the planes of every expert of a layer of R choices over at most umax experts, packed: at most R + 127 umax padded
// activations (tiles of up to 128), each expert's two planes rounded up to 256 bytes
size_t moe_ws_bytes(int cols, int R, int umax) {
    const size_t nbk = cols / 256, rows = (size_t)R + 127 * (size_t)umax;
    return nbk * rows * (256 + 36) + 2 * 256 * (size_t)umax;
}

// one product's family and launch: rows x cols weights of `type`, umax expert slots of `njob` products each, R choices
struct MoeLaunch {
    esq::MoeFamily F{};
    MvLaunch L{};
    int bn = 0, grid = 0, njobs = 0, nprep = 0;   // tile upper bound; job table entries; pre-pass entries (MM)
    long items = 0;                               // pre-pass item upper bound (MM)
};

int moe_family(es_hip_moe_ctx *c, uint32_t type, int rows, int cols, int umax, int njob, int R, double expect, int maxc,
               const uint8_t *w0, const uint8_t *act, const int *arow, uint64_t astride, float *y, uint64_t ystride,
               uint8_t *ws, MoeLaunch &M, bool gated = false) {
    FmtInfo f;
    fmt_info(type, f);
    const int nbk = cols / f.be;
    M.F = esq::MoeFamily{};
    M.njobs = njob * umax + 1;
    M.nprep = umax + 1;
    int bn = 0;
    // activation rows: the layer's tokens (gate/up, gathered) or its pair rows (down)
    if (moe_mx_family(type, rows, cols, expect, R, arow ? (size_t)std::max(maxc, 1) : (size_t)R, astride, ystride)) {
        M.F.kind = esq::MOE_FAM_MX;
        M.F.gated = gated ? 1 : 0;
        const int trows = gated ? 256 : esq::MX_ROWS;   // the gated kernel's tiles are one block of h
        const int row_tiles = (rows + trows - 1) / trows;
        M.F.mx_tiles = row_tiles;
        M.F.row_tiles8 = 8 * ((row_tiles + 7) / 8);
        esq::MkJob &j = M.F.mk;
        j.W = w0;
        j.act = act;
        j.arow = arow;
        j.y = y;
        j.astride = astride;
        j.ystride = ystride;
        j.row_bytes = (uint64_t)nbk * f.bb;
        j.r0 = 0;
        j.r1 = rows;
        j.cols = cols;
        j.na = 0;
        j.tile0 = 0;
        j.ntok_tiles = 1;
        // sum over experts of ceil(count / MX_TOK) activation tiles, each at most row_tiles8 tiles
        M.grid = njob * M.F.row_tiles8 * ((R + esq::MX_TOK - 1) / esq::MX_TOK + umax);
        return ES_HIP_OK;
    }
    if (ws && moe_mm_family(type, cols, expect, bn)) {
        M.F.kind = esq::MOE_FAM_MM;
        M.bn = M.F.bn = bn;
        const int row_tiles = (rows + 127) / 128;
        M.F.row_tiles8 = 8 * ((row_tiles + 7) / 8);
        esq::MmJob &j = M.F.mm;
        j.W = w0;
        j.xq = ws;
        j.xm = ws;
        j.y = y;
        j.ystride = ystride;
        j.row_bytes = (uint64_t)nbk * f.bb;
        j.r0 = 0;
        j.r1 = rows;
        j.cols = cols;
        j.ntok_tiles = 1;
        esq::PrepJob &p = M.F.pj;
        p.act = act;
        p.arow = arow;
        p.xq = ws;
        p.xm = ws;
        p.astride = astride;
        p.nbk = nbk;
        p.kind = 2;
        const long ntok_ub = (R + bn - 1) / bn + umax;   // sum over experts of ceil(count / bn)
        M.grid = njob * M.F.row_tiles8 * (int)ntok_ub;
        M.items = ntok_ub * bn * nbk * (long)esq::prep_words(2) + (long)umax * esq::PREP_SPAN;
        return ES_HIP_OK;
    }
    // the decode kernel, sized as the planner sizes umax * njob products of about `expect` activations each (the sizing
    // depends on the shapes only: kept per context). The activations per pass cover the counts routing can produce: an
    // expert takes at most maxc (the layer's tokens) and usually a few more than the mean, so the planner's four-wide pass
    // whenever three or more are possible (sized at the mean, 32 tokens over 128 experts ran two-wide passes and lost
    // 11.6 us per layer re-reading the weights of the experts above it)
    M.F.kind = esq::MOE_FAM_MV;
    const int na = std::min(std::max(1, maxc), std::max(4, (int)std::ceil(expect)));
    const std::array<int, 6> key{(int)type, rows, cols, umax, njob, na};
    auto it = c->mv_cache.find(key);
    if (it == c->mv_cache.end()) {
        std::vector<Req> reqs((size_t)umax * njob,
                              Req{type, w0, act, y, nullptr, nullptr, 0, rows, cols, na, astride, ystride, arow, 1});
        std::vector<Group> groups;
        if (int rc = plan_groups(reqs, groups)) return rc;
        if (groups.size() != 1) return fail(ES_HIP_EINVAL, "MoE product planned as %zu launches", groups.size());
        it = c->mv_cache.emplace(key, std::make_pair(groups[0].L, groups[0].jobs[0])).first;
    }
    M.L = it->second.first;
    M.F.mv = it->second.second;   // this call's pointers: the template must point at live buffers (empty jobs keep them)
    M.F.mv.W = w0;
    M.F.mv.act = act;
    M.F.mv.arow = arow;
    M.F.mv.astride = astride;
    M.F.mv.y = y;
    M.F.mv.ystride = ystride;
    M.F.mv.na = 0;
    M.F.mv.tile0 = 0;
    M.F.mv_tiles = (rows + M.F.mv.rows_per_wg - 1) / M.F.mv.rows_per_wg;
    M.grid = M.L.grid = njob * umax * M.F.mv_tiles;
    M.L.nt = 0;   // each expert's job takes the width of its own count (the grouping sets it, at most the template's)
    return ES_HIP_OK;
}

}  // namespace

extern "C" {

es_hip_moe_ctx *es_hip_moe_ctx_create(const es_hip_moe *m, int max_tokens, int k) {
    if (need_device()) return nullptr;
    if (!m) { fail(ES_HIP_EINVAL, "null MoE description"); return nullptr; }
    FmtInfo fg, fu, fd;
    if (!fmt_info(m->gate_type, fg) || !fmt_info(m->up_type, fu) || !fmt_info(m->down_type, fd)) {
        fail(ES_HIP_EINVAL, "an expert type is not computed by this library");
        return nullptr;
    }
    if (m->gate_type != m->up_type) { fail(ES_HIP_EINVAL, "the device-routed MoE needs gate and up of one type"); return nullptr; }
    if (m->n <= 0 || m->ff <= 0 || m->n % fg.be || m->ff % fd.be) { fail(ES_HIP_EINVAL, "bad widths n %d, ff %d", m->n, m->ff); return nullptr; }
    if (m->n_exp <= 0 || m->n_exp > esq::ROUTE_MAX_EXPERTS || !m->gate || !m->up || !m->down) {
        fail(ES_HIP_EINVAL, "bad expert table (1 to %d experts)", esq::ROUTE_MAX_EXPERTS);
        return nullptr;
    }
    if (max_tokens <= 0 || k <= 0 || k > 64 || k > m->n_exp || (long)max_tokens * k > esq::MOE_MAX_PAIRS) {
        fail(ES_HIP_EINVAL, "bad max_tokens %d or k %d (at most %d choices)", max_tokens, k, esq::MOE_MAX_PAIRS);
        return nullptr;
    }
    auto *c = new es_hip_moe_ctx();
    c->gt = m->gate_type; c->ut = m->up_type; c->dt = m->down_type;
    c->n = m->n; c->ff = m->ff; c->n_exp = m->n_exp; c->max_tokens = max_tokens; c->k = k;
    c->h_q8k = fd.be == 256;
    c->hstride = (uint64_t)(m->ff / fd.be) * fd.ab;
    std::vector<const uint8_t *> hg(m->n_exp), hu(m->n_exp), hd(m->n_exp);
    for (int e = 0; e < m->n_exp; e++) {
        hg[e] = static_cast<const uint8_t *>(m->gate[e]);
        hu[e] = static_cast<const uint8_t *>(m->up[e]);
        hd[e] = static_cast<const uint8_t *>(m->down[e]);
        if (!c->w_gate0 && hg[e] && hu[e] && hd[e]) { c->w_gate0 = hg[e]; c->w_down0 = hd[e]; }
    }
    if (!c->w_gate0) { fail(ES_HIP_EINVAL, "no expert has weights"); delete c; return nullptr; }
    for (int e = 0; e < m->n_exp; e++)   // experts without weights point at one that has them (they must not be routed)
        if (!hg[e] || !hu[e] || !hd[e]) { hg[e] = hu[e] = c->w_gate0; hd[e] = c->w_down0; }
    const int R = max_tokens * k, umax = std::min(m->n_exp, R), n = m->n, ff = m->ff;
    const bool gu_mm = m->gate_type == ES_HIP_Q2_K || m->gate_type == ES_HIP_Q4_K || m->gate_type == ES_HIP_Q6_K;
    const bool dn_mm = m->down_type == ES_HIP_Q2_K || m->down_type == ES_HIP_Q4_K || m->down_type == ES_HIP_Q6_K;
    c->gu_slot = gu_mm ? moe_ws_bytes(n, R, umax) : 0;
    c->dn_slot = dn_mm ? moe_ws_bytes(ff, R, umax) : 0;
    const size_t job = std::max({sizeof(MvJob), sizeof(esq::MmJob), sizeof(esq::MkJob)});
    size_t off = 0;
    auto take = [&](size_t bytes) { const size_t o = off; off += align256(std::max<size_t>(bytes, 1)); return o; };
    const size_t o_sel = take(sizeof(int) * R), o_w = take(sizeof(float) * R), o_tok = take(sizeof(int) * R),
                 o_rowof = take(sizeof(int) * R), o_wv = take(sizeof(float) * R), o_kk = take(sizeof(int) * max_tokens),
                 o_g = take(sizeof(void *) * m->n_exp), o_u = take(sizeof(void *) * m->n_exp), o_d = take(sizeof(void *) * m->n_exp),
                 o_bgu = take(sizeof(float) * 2 * ff * (size_t)R), o_ha = take(c->hstride * R), o_bye = take(sizeof(float) * n * (size_t)R),
                 o_guj = take(job * (2 * (size_t)umax + 1)), o_dnj = take(job * ((size_t)umax + 1)),
                 o_gup = take(sizeof(esq::PrepJob) * (umax + 1)), o_dnp = take(sizeof(esq::PrepJob) * (umax + 1)),
                 o_guw = take(c->gu_slot), o_dnw = take(c->dn_slot);
    hipError_t e = hipMalloc(&c->buf, off);
    if (e != hipSuccess) { hip_fail(e, "hipMalloc (MoE context)"); delete c; return nullptr; }
    uint8_t *b = c->buf;
    c->sel = reinterpret_cast<int *>(b + o_sel);
    c->w = reinterpret_cast<float *>(b + o_w);
    c->tok_of = reinterpret_cast<int *>(b + o_tok);
    c->rowof = reinterpret_cast<int *>(b + o_rowof);
    c->wv = reinterpret_cast<float *>(b + o_wv);
    c->kk = reinterpret_cast<int *>(b + o_kk);
    c->dgate = reinterpret_cast<const uint8_t **>(b + o_g);
    c->dup = reinterpret_cast<const uint8_t **>(b + o_u);
    c->ddown = reinterpret_cast<const uint8_t **>(b + o_d);
    c->bgu = reinterpret_cast<float *>(b + o_bgu);
    c->ha = b + o_ha;
    c->bye = reinterpret_cast<float *>(b + o_bye);
    c->gu_jobs = b + o_guj;
    c->dn_jobs = b + o_dnj;
    c->gu_prep = reinterpret_cast<esq::PrepJob *>(b + o_gup);
    c->dn_prep = reinterpret_cast<esq::PrepJob *>(b + o_dnp);
    c->gu_ws = gu_mm ? b + o_guw : nullptr;
    c->dn_ws = dn_mm ? b + o_dnw : nullptr;
    std::vector<int> kk(max_tokens, k);
    if ((e = hipMemcpy(c->kk, kk.data(), sizeof(int) * max_tokens, hipMemcpyHostToDevice)) != hipSuccess ||
        (e = hipMemcpy(c->dgate, hg.data(), sizeof(void *) * m->n_exp, hipMemcpyHostToDevice)) != hipSuccess ||
        (e = hipMemcpy(c->dup, hu.data(), sizeof(void *) * m->n_exp, hipMemcpyHostToDevice)) != hipSuccess ||
        (e = hipMemcpy(c->ddown, hd.data(), sizeof(void *) * m->n_exp, hipMemcpyHostToDevice)) != hipSuccess ||
        (e = hipMemset(c->bye, 0, sizeof(float) * n)) != hipSuccess) {
        hip_fail(e, "MoE context set-up");
        (void)hipFree(c->buf);
        delete c;
        return nullptr;
    }
    return c;
}

void es_hip_moe_ctx_destroy(es_hip_moe_ctx *c) {
    if (!c) return;
    if (c->buf) (void)hipFree(c->buf);
    delete c;
}

}  // extern "C"

namespace {

// one layer from a routing already in the context's sel / w (device), in stream order
int moe_ctx_layer(es_hip_moe_ctx *c, int N, const void *x, size_t xstride, float *out, size_t ostride, hipStream_t s) {
    const int R = N * c->k, umax = std::min(c->n_exp, R), n = c->n, ff = c->ff;
    FmtInfo fg, fd;
    fmt_info(c->gt, fg);
    fmt_info(c->dt, fd);
    const uint64_t xs = xstride ? xstride : (uint64_t)(n / fg.be) * fg.ab;
    const double expect = (double)R / umax;   // choices per expert if every slot were used
    MoeLaunch G, D;
    // Q2_K gate and up with a K-quant down on the gated expert kernel: one job per expert slot, h written as Q8_K blocks
    const bool gated = g_moe_gated.load() && c->gt == ES_HIP_Q2_K && c->h_q8k && ff % 256 == 0 &&
                       moe_mx_family(c->gt, ff, n, expect, R, (size_t)std::max(N, 1), xs, c->hstride);
    if (gated) {
        if (int rc = moe_family(c, c->gt, ff, n, umax, 1, R, expect, N, c->w_gate0, static_cast<const uint8_t *>(x), c->tok_of,
                                xs, reinterpret_cast<float *>(c->ha), c->hstride, c->gu_ws, G, true))
            return rc;
    } else if (int rc = moe_family(c, c->gt, ff, n, umax, 2, R, expect, N, c->w_gate0, static_cast<const uint8_t *>(x),
                                   c->tok_of, xs, c->bgu, 2 * (uint64_t)ff, c->gu_ws, G)) {
        return rc;
    }
    if (int rc = moe_family(c, c->dt, n, ff, umax, 1, R, expect, N, c->w_down0, c->ha, nullptr, c->hstride, c->bye, (uint64_t)n,
                            c->dn_ws, D))
        return rc;
    esq::MoeDevArgs a{};
    a.sel = c->sel;
    a.w = c->w;
    a.ntok = N;
    a.k = c->k;
    a.n_exp = c->n_exp;
    a.umax = umax;
    a.ff = ff;
    a.n = n;
    a.gate = c->dgate;
    a.up = c->dup;
    a.down = c->ddown;
    a.x = static_cast<const uint8_t *>(x);
    a.xstride = xs;
    a.hstride = c->hstride;
    a.bgu = c->bgu;
    a.ha = c->ha;
    a.bye = c->bye;
    a.tok_of = c->tok_of;
    a.rowof = c->rowof;
    a.wv = c->wv;
    a.gu_jobs = c->gu_jobs;
    a.dn_jobs = c->dn_jobs;
    a.gu_prep = c->gu_prep;
    a.dn_prep = c->dn_prep;
    a.gu_ws = c->gu_ws;
    a.dn_ws = c->dn_ws;
    hipError_t e = esq::moe_group_build_launch(a, G.F, D.F, s);
    if (e != hipSuccess) return hip_fail(e, "MoE grouping launch");
    const int order = g_order.load();
    auto run = [&](const MoeLaunch &M, uint32_t type, void *jobs, esq::PrepJob *prep) -> int {
        if (M.F.kind == esq::MOE_FAM_MV) {
            e = esq::mv_launch(M.L, static_cast<const MvJob *>(jobs), M.njobs, M.F.mv, order, s);
            return e == hipSuccess ? ES_HIP_OK : hip_fail(e, "MoE decode-kernel launch");
        }
        if (M.F.kind == esq::MOE_FAM_MX) {
            e = M.F.gated ? esq::mxg_launch(M.F.mk.arow != nullptr, M.F.mk.cols / 256, static_cast<const esq::MkJob *>(jobs),
                                            M.njobs, M.F.mk, M.grid, order, s)
                          : esq::mx_launch((int)type, M.F.mk.arow != nullptr, M.F.mk.cols / 256,
                                           static_cast<const esq::MkJob *>(jobs), M.njobs, M.F.mk, M.grid, order, s);
            return e == hipSuccess ? ES_HIP_OK : hip_fail(e, "MoE expert-kernel launch");
        }
        if ((e = esq::prep_launch(prep, M.nprep, M.F.pj, M.items, s)) != hipSuccess) return hip_fail(e, "MoE pre-pass launch");
        e = esq::mm_launch((int)type, 128, M.bn, 8, static_cast<const esq::MmJob *>(jobs), M.njobs, M.F.mm, M.grid, order, s);
        return e == hipSuccess ? ES_HIP_OK : hip_fail(e, "MoE matrix-core launch");
    };
    if (int rc = run(G, c->gt, c->gu_jobs, c->gu_prep)) return rc;
    if (!G.F.gated && (e = esq::moe_swiglu_launch(c->bgu, R, ff, c->h_q8k, c->ha, c->hstride, s)) != hipSuccess)
        return hip_fail(e, "SwiGLU launch");
    if (int rc = run(D, c->dt, c->dn_jobs, c->dn_prep)) return rc;
    e = esq::moe_combine_launch(c->bye, c->rowof, c->wv, c->kk, c->k, N, n, out, ostride ? ostride : (uint64_t)n, s);
    return e == hipSuccess ? ES_HIP_OK : hip_fail(e, "combine launch");
}

int moe_ctx_check(const es_hip_moe_ctx *c, int N, const void *x, const float *out, size_t ostride) {
    if (!c) return fail(ES_HIP_EINVAL, "null MoE context");
    if (N < 0 || N > c->max_tokens) return fail(ES_HIP_EINVAL, "N %d outside [0, %d]", N, c->max_tokens);
    if (N > 0 && (!x || !out)) return fail(ES_HIP_EINVAL, "null activations or outputs");
    if (N > 1 && ostride && ostride < (size_t)c->n) return fail(ES_HIP_EINVAL, "ostride %zu < n %d", ostride, c->n);
    return ES_HIP_OK;
}
// the token rows x as check_req checks a product's activations: dword-aligned rows at least one row's blocks apart
int moe_ctx_check_x(const es_hip_moe_ctx *c, int N, const void *x, size_t xstride) {
    if (N == 0) return ES_HIP_OK;
    FmtInfo fg;
    fmt_info(c->gt, fg);
    const size_t packed = (size_t)(c->n / fg.be) * fg.ab;
    if ((reinterpret_cast<uintptr_t>(x) & 3) || (xstride & 3))
        return fail(ES_HIP_EINVAL, "activation rows must be 4-byte aligned (pointer and stride)");
    if (N > 1 && xstride && xstride < packed)
        return fail(ES_HIP_EINVAL, "activation stride %zu < %zu bytes of one token's blocks", xstride, packed);
    return ES_HIP_OK;
}

}  // namespace

extern "C" {

int es_hip_moe_ctx_run_logits(es_hip_moe_ctx *c, int N, const float *logits, size_t lstride, int norm_topk, const void *x,
                              size_t xstride, float *out, size_t ostride, int *sel_out, float *w_out, void *stream) {
    if (int rc = need_device()) return rc;
    if (int rc = moe_ctx_check(c, N, x, out, ostride)) return rc;
    if (int rc = moe_ctx_check_x(c, N, x, xstride)) return rc;
    if (N == 0) return ES_HIP_OK;
    if (!logits) return fail(ES_HIP_EINVAL, "null logits");
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e = esq::route_softmax_launch(logits, lstride ? lstride : (uint64_t)c->n_exp, N, c->n_exp, c->k, norm_topk,
                                             c->sel, c->w, c->k, s);
    if (e != hipSuccess) return hip_fail(e, "routing launch");
    const size_t pairs = (size_t)N * c->k;
    if (sel_out && (e = hipMemcpyAsync(sel_out, c->sel, pairs * sizeof(int), hipMemcpyDeviceToDevice, s)) != hipSuccess)
        return hip_fail(e, "routing copy");
    if (w_out && (e = hipMemcpyAsync(w_out, c->w, pairs * sizeof(float), hipMemcpyDeviceToDevice, s)) != hipSuccess)
        return hip_fail(e, "routing copy");
    return moe_ctx_layer(c, N, x, xstride, out, ostride, s);
}

int es_hip_moe_ctx_run(es_hip_moe_ctx *c, int N, const int *sel, const float *w, const void *x, size_t xstride, float *out,
                       size_t ostride, void *stream) {
    if (int rc = need_device()) return rc;
    if (int rc = moe_ctx_check(c, N, x, out, ostride)) return rc;
    if (int rc = moe_ctx_check_x(c, N, x, xstride)) return rc;
    if (N == 0) return ES_HIP_OK;
    if (!sel || !w) return fail(ES_HIP_EINVAL, "null routing");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const size_t pairs = (size_t)N * c->k;
    hipError_t e;
    if ((e = hipMemcpyAsync(c->sel, sel, pairs * sizeof(int), hipMemcpyDeviceToDevice, s)) != hipSuccess ||
        (e = hipMemcpyAsync(c->w, w, pairs * sizeof(float), hipMemcpyDeviceToDevice, s)) != hipSuccess)
        return hip_fail(e, "routing copy");
    return moe_ctx_layer(c, N, x, xstride, out, ostride, s);
}

}  // extern "C"

namespace {
// Checks of an activation preparation's block outputs (either may be null); fills in packed strides.
int prep_blocks(int rows, int cols, const void *q80, size_t &q80s, const void *q8k, size_t &q8ks) {
    if (rows < 0 || cols <= 0) return fail(ES_HIP_EINVAL, "bad shape: %d rows of %d values", rows, cols);
    if (q80) {
        const size_t packed = (size_t)(cols / 32) * 36;
        if (cols % 32) return fail(ES_HIP_EINVAL, "Q8_0 blocks need cols %% 32 == 0 (cols %d)", cols);
        if (!q80s) q80s = packed;
        if (rows > 1 && q80s < packed) return fail(ES_HIP_EINVAL, "Q8_0 stride %zu < %zu bytes of one row", q80s, packed);
        if ((reinterpret_cast<uintptr_t>(q80) & 3) || (q80s & 3)) return fail(ES_HIP_EINVAL, "Q8_0 blocks must be 4-byte aligned");
    }
    if (q8k) {
        const size_t packed = (size_t)(cols / 256) * 292;
        if (cols % 256) return fail(ES_HIP_EINVAL, "Q8_K blocks need cols %% 256 == 0 (cols %d)", cols);
        if (!q8ks) q8ks = packed;
        if (rows > 1 && q8ks < packed) return fail(ES_HIP_EINVAL, "Q8_K stride %zu < %zu bytes of one row", q8ks, packed);
        if ((reinterpret_cast<uintptr_t>(q8k) & 3) || (q8ks & 3)) return fail(ES_HIP_EINVAL, "Q8_K blocks must be 4-byte aligned");
    }
    return ES_HIP_OK;
}
// a float row array: pointer, stride (0: packed) and row length
int prep_floats(const char *what, const float *p, size_t &stride, int rows, size_t len) {
    if (!stride) stride = len;
    if (rows > 1 && stride < len) return fail(ES_HIP_EINVAL, "%s stride %zu < %zu floats of one row", what, stride, len);
    if (reinterpret_cast<uintptr_t>(p) & 3) return fail(ES_HIP_EINVAL, "%s must be 4-byte aligned", what);
    return ES_HIP_OK;
}
}  // namespace

extern "C" {

int es_hip_act_prepare_dev(const float *x, size_t xstride, int rows, int cols, void *q80, size_t q80_stride, void *q8k,
                           size_t q8k_stride, void *stream) {
    if (int rc = need_device()) return rc;
    if (int rc = prep_blocks(rows, cols, q80, q80_stride, q8k, q8k_stride)) return rc;
    if (!q80 && !q8k) return fail(ES_HIP_EINVAL, "no output blocks asked for");
    if (rows == 0) return ES_HIP_OK;
    if (!x) return fail(ES_HIP_EINVAL, "null x");
    if (int rc = prep_floats("x", x, xstride, rows, (size_t)cols)) return rc;
    hipError_t e = esq::act_prep_launch(x, xstride, rows, cols, static_cast<uint8_t *>(q80), q80_stride,
                                        static_cast<uint8_t *>(q8k), q8k_stride, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? ES_HIP_OK : hip_fail(e, "activation preparation launch");
}

int es_hip_rmsnorm_prepare_dev(const float *x, size_t xstride, const float *w, float eps, int rows, int cols, float *xn,
                               size_t xn_stride, void *q80, size_t q80_stride, void *q8k, size_t q8k_stride, void *stream) {
    if (int rc = need_device()) return rc;
    if (int rc = prep_blocks(rows, cols, q80, q80_stride, q8k, q8k_stride)) return rc;
    if (!xn && !q80 && !q8k) return fail(ES_HIP_EINVAL, "no output asked for");
    if (cols > esq::ACT_RMS_MAX_COLS || cols % 32)
        return fail(ES_HIP_EINVAL, "rmsnorm rows of %d values: a multiple of 32 up to %d is needed", cols, esq::ACT_RMS_MAX_COLS);
    if (rows == 0) return ES_HIP_OK;
    if (!x) return fail(ES_HIP_EINVAL, "null x");
    if (int rc = prep_floats("x", x, xstride, rows, (size_t)cols)) return rc;
    if (xn)
        if (int rc = prep_floats("xn", xn, xn_stride, rows, (size_t)cols)) return rc;
    if (reinterpret_cast<uintptr_t>(w) & 3) return fail(ES_HIP_EINVAL, "w must be 4-byte aligned");
    hipError_t e = esq::act_prep_rms_launch(x, xstride, w, eps, rows, cols, xn, xn_stride, static_cast<uint8_t *>(q80),
                                            q80_stride, static_cast<uint8_t *>(q8k), q8k_stride,
                                            static_cast<hipStream_t>(stream));
    return e == hipSuccess ? ES_HIP_OK : hip_fail(e, "rmsnorm preparation launch");
}

int es_hip_swiglu_prepare_dev(const float *gu, size_t gu_stride, int rows, int ff, float *h, size_t h_stride, void *q80,
                              size_t q80_stride, void *q8k, size_t q8k_stride, void *stream) {
    if (int rc = need_device()) return rc;
    if (int rc = prep_blocks(rows, ff, q80, q80_stride, q8k, q8k_stride)) return rc;
    if (!h && !q80 && !q8k) return fail(ES_HIP_EINVAL, "no output asked for");
    if (rows == 0) return ES_HIP_OK;
    if (!gu) return fail(ES_HIP_EINVAL, "null gate|up rows");
    if (int rc = prep_floats("gate|up", gu, gu_stride, rows, 2 * (size_t)ff)) return rc;
    if (h)
        if (int rc = prep_floats("h", h, h_stride, rows, (size_t)ff)) return rc;
    hipError_t e = esq::act_prep_swiglu_launch(gu, gu_stride, rows, ff, h, h_stride, static_cast<uint8_t *>(q80), q80_stride,
                                               static_cast<uint8_t *>(q8k), q8k_stride, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? ES_HIP_OK : hip_fail(e, "SwiGLU preparation launch");
}

int es_hip_dequant_row_dev(uint32_t type, const void *src, float *dst, long n, void *stream) {
    if (int rc = need_device()) return rc;
    FmtInfo f;
    if (!fmt_info(type, f)) return fail(ES_HIP_EINVAL, "type %u is not computed by this library", type);
    if (n < 0 || n % f.be) return fail(ES_HIP_EINVAL, "n = %ld is not a whole number of %d-element blocks", n, f.be);
    if (n == 0) return ES_HIP_OK;
    if (!src || !dst) return fail(ES_HIP_EINVAL, "null source or output");
    if (reinterpret_cast<uintptr_t>(dst) & 3) return fail(ES_HIP_EINVAL, "dst must be 4-byte aligned");
    hipError_t e = esq::dequant_launch(type, src, dst, n, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? ES_HIP_OK : hip_fail(e, "dequant launch");
}

int es_hip_matvec_float_dev(uint32_t type, const void *W, int cols, int r0, int r1, const float *x, size_t xstride, int na,
                            float *y, size_t ystride, void *stream) {
    if (int rc = need_device()) return rc;
    FmtInfo f;
    if (!fmt_info(type, f)) return fail(ES_HIP_EINVAL, "type %u is not computed by this library", type);
    if (cols <= 0 || cols % f.be) return fail(ES_HIP_EINVAL, "type %u: cols %d is not a positive multiple of %d", type, cols, f.be);
    if (r0 < 0 || r1 < r0 || na < 0) return fail(ES_HIP_EINVAL, "bad row range [%d, %d) or activation count %d", r0, r1, na);
    if (r1 == r0 || na == 0) return ES_HIP_OK;
    if (!W || !x || !y) return fail(ES_HIP_EINVAL, "null W, x or y");
    if (reinterpret_cast<uintptr_t>(W) & 1) return fail(ES_HIP_EINVAL, "W must be 2-byte aligned");
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 3) return fail(ES_HIP_EINVAL, "x and y must be 4-byte aligned");
    if (!xstride) xstride = (size_t)cols;
    if (na > 1 && xstride < (size_t)cols) return fail(ES_HIP_EINVAL, "x stride %zu < cols %d", xstride, cols);
    if (na > 1 && ystride < (size_t)r1) return fail(ES_HIP_EINVAL, "ystride %zu < r1 %d: outputs of activations overlap", ystride, r1);
    if (na > 65535 * 8) return fail(ES_HIP_EINVAL, "%d activations in one call (at most %d)", na, 65535 * 8);
    const size_t rb = (size_t)(cols / f.be) * f.bb;
    hipError_t e = esq::fdot_launch(type, W, rb, r0, r1, cols, x, xstride, na, y, ystride, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? ES_HIP_OK : hip_fail(e, "float-path launch");
}

int es_hip_route_softmax_dev(const float *logits, size_t lstride, int ntok, int n_exp, int k, int norm_topk, int *sel, float *w,
                             int kmax, void *stream) {
    if (int rc = need_device()) return rc;
    if (ntok < 0 || n_exp <= 0 || n_exp > esq::ROUTE_MAX_EXPERTS || k <= 0 || k > 64 || k > n_exp || kmax < k)
        return fail(ES_HIP_EINVAL, "bad routing shape: %d tokens, %d experts, top %d of rows of %d", ntok, n_exp, k, kmax);
    if (ntok == 0) return ES_HIP_OK;
    if (!logits || !sel || !w) return fail(ES_HIP_EINVAL, "null logits, sel or w");
    if (!lstride) lstride = (size_t)n_exp;
    if (ntok > 1 && lstride < (size_t)n_exp) return fail(ES_HIP_EINVAL, "logit stride %zu < %d", lstride, n_exp);
    if ((reinterpret_cast<uintptr_t>(logits) | reinterpret_cast<uintptr_t>(sel) | reinterpret_cast<uintptr_t>(w)) & 3)
        return fail(ES_HIP_EINVAL, "logits, sel and w must be 4-byte aligned");
    hipError_t e = esq::route_softmax_launch(logits, lstride, ntok, n_exp, k, norm_topk, sel, w, kmax,
                                             static_cast<hipStream_t>(stream));
    return e == hipSuccess ? ES_HIP_OK : hip_fail(e, "routing launch");
}

int es_hip_swiglu_dev(const float *g, const float *u, float *h, long n, void *stream) {
    if (int rc = need_device()) return rc;
    if (n < 0 || (n > 0 && (!g || !u || !h))) return fail(ES_HIP_EINVAL, "bad SwiGLU arguments");
    hipError_t e = esq::swiglu_plain_launch(g, u, h, n, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? ES_HIP_OK : hip_fail(e, "SwiGLU launch");
}

}  // extern "C"
