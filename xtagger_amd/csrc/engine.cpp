// engine.cpp - the wd / EVA02-L engine behind the reference's C host API (src/engine/eva.h:573-745), on HIP for one
// MI355X. eva_open returns at once; the bring-up (device, weights, packing, buffers, graph capture) runs on its own
// thread and eva_ready joins it. One forward = one replay of a HIP graph captured once for nb inputs (eva.h:531-536).
// A batch of nb inputs runs as two halves at once, on two lanes with their own activations, stream and graph (images
// 0 .. ceil(nb / 2) - 1 on lane 0, the engine stream, the rest on lane 1): each half fills the CUs that the other's
// short last rounds of tiles leave idle. Input and score buffers are shared, each lane using its slice.
#include <hip/hip_runtime.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <vector>

#include "xt_abi.h"
#include "xt_stream.h"
#include "xtag_eva.h"


#define V2_HIDP 2736          // hidden padding of the reference's v2 blob (export_eva.py:19)
#define EVA_HB_OFF (-16.0f)   // bias of an extra head row nothing has written (eva.h:69)
#define EV_HPUT_SLOTS 256     // eva_head_put rows staged at once before a call waits for the oldest copy
#define EV_HPUT_SLOT 2304     // bytes per slot: 1024 fp16 weights, then the fp32 bias (256-byte multiple)

#define V3_NS 12              // v3 scale table columns per layer: wdq x4, adq x4, q, k, v, pad (eva.h:379)

struct Layer {
    const float *ln1w, *ln1b, *ln2w, *ln2b, *mlnw, *mlnb;  // in the blob
    const uint16_t *wqkv16, *wo16, *w1216, *w216;          // v2: fp16 block weights in the blob
    const uint8_t *wqkv8, *wo8, *w128, *w28;               // v3: E4M3 block weights in the blob, one scale each
    const float *rs0, *cn0, *dn0;                          // v3: h multipliers [2736], fold terms c, d [1024]
    float *rs;                                             // v3: rs padded to 2816 units (zeros past 2736)
    uint8_t *wqkv, *wo, *w12, *w2;                         // packed E4M3 (2:4-pruned with EVA_SPARSE24)
    float *sqkv, *so, *s12, *s2, *cn, *dn;
    uint8_t *vqkv, *vo, *v12, *v2;                         // EVA_SPARSE24: pack24 values of the pruned weights
    uint32_t *xqkv, *xo, *x12, *x2;                        // and their indices
    size_t end;                                            // blob offset past the layer's last tensor
};

struct eva_impl {
    int devno, bstatus, up, booted;
    uint32_t flags;                                        // EVA_SPARSE24
    uint32_t ver;                                          // blob version: 2 (fp16 weights) or 3 (E4M3 + scales)
    float tab[EVA_NL * V3_NS];                             // v3 scale table (host copy, eva.h:379-428)
    pthread_t boot;
    char *path;                                            // own copy of the weights path
    size_t wbytes;
    uint32_t nb;                                           // inputs per launch
    uint32_t nl, lnb[2], loff[2];                          // lanes (1 when nb = 1); each lane's inputs and first one
    uint32_t cnb, cM, cMp;                                 // the lane ev_forward works on: inputs, rows, padded rows
    hipStream_t st;
    uint8_t *blob;                                         // the file's tensors, resident
    const uint16_t *pe;
    const float *pos, *cs, *fnw, *fnb, *hb0;
    const uint16_t *hw0;
    Layer L[EVA_NL];
    uint16_t *hmaster;                                     // head fp16 [nt][1024] (file rows, then extra rows)
    float *hb;                                             // [nt]
    uint8_t *hq;                                           // head E4M3 [nt][1024], each row with its own scales
    float *hs;                                             // 1x128 scale planes [8][ldh]
    uint32_t ldh;                                          // nt rounded up to 64
    uint8_t *hput;                                         // pinned staging slots of eva_head_put (row + bias)
    hipEvent_t hput_ev[EV_HPUT_SLOTS];                     // the last copy out of each slot
    uint32_t hput_next;
    float *scratch;
    // activations of the lane ev_forward works on (lane 0 outside graph capture)
    uint16_t *in, *x, *q, *k, *vt, *pn;
    uint8_t *h8, *m8, *pq;
    float *sh, *sm, *stat, *pool, *ps, *out;
    hipGraphExec_t graph;
    struct Acts {
        uint16_t *in, *x, *q, *k, *vt, *pn;
        uint8_t *h8, *m8, *pq;
        float *sh, *sm, *stat, *pool, *ps, *out;
    } act[2];
    uint16_t *in_all, *pn_all;                             // inputs [nb][1024][592], head inputs [nb][1024]
    float *out_all;                                        // scores [nb][nt]
    hipStream_t lst[2];                                    // lane streams (lst[0] = st)
    hipGraphExec_t lgraph[2];                              // lane graphs (lgraph[0] = graph)
    hipEvent_t lane_ev;                                    // after lane 1's half of the last batch
    hipEvent_t head_ev;                                    // after the last eva_head_put's update (on st)
    // eva_profile: an event after every op of one direct forward (eva.h:71-88, 312-338), 172 ops per half at 24
    // layers
    hipEvent_t pev[512];
    uint8_t pid[512];
    int pk, pon;
    hipEvent_t done[EVA_NBUF];
    uint16_t *stage[EVA_NBUF];                             // pinned staging of each buf's inputs (at its first submit)
    std::vector<void *> allocs;
};

static int ev_alloc(eva_impl *E, void **p, size_t bytes, bool zero)
{
    if (hipMalloc(p, bytes ? bytes : 16) != hipSuccess) return xt_fail("hipMalloc", "out of device memory");
    E->allocs.push_back(*p);
    if (zero && hipMemset(*p, 0, bytes) != hipSuccess) return xt_fail("hipMemset", "failed");
    return 0;
}
#define EV_ALLOC(E, p, bytes, zero)                                    \
    do {                                                               \
        void *tmp_;                                                    \
        if (ev_alloc((E), &tmp_, (bytes), (zero))) return -1;          \
        (p) = (decltype(p))tmp_;                                       \
    } while (0)
#define EV_CK(call)                                                    \
    do {                                                               \
        if ((call)) return -1;                                         \
    } while (0)

// Blob layout of export_eva.py (eva.h:380-430): every tensor on a 256-byte boundary. v3 leads with the [24][12]
// scale table and stores the block weights as E4M3 bytes, with rs | W~2 | c | d in place of the MLP LN's gamma | beta
// | W2.
static int ev_layout(eva_impl *E, uint32_t ntp)
{
    size_t off = 0;
    auto take = [&](size_t bytes) -> uint8_t * {
        off = (off + 255) & ~(size_t)255;
        uint8_t *p = E->blob + off;
        off += bytes;
        return p;
    };
    const bool v3 = E->ver == 3;
    if (v3) take((size_t)EVA_NL * V3_NS * 4);
    E->pe = (const uint16_t *)take((size_t)EVA_D * EVA_K0P * 2);
    E->pos = (const float *)take((size_t)EVA_T * EVA_D * 4);
    E->cs = (const float *)take((size_t)EVA_NP * 32 * 2 * 4);
    for (int i = 0; i < EVA_NL; i++) {
        Layer &L = E->L[i];
        L.ln1w = (const float *)take(EVA_D * 4);
        L.ln1b = (const float *)take(EVA_D * 4);
        if (v3) {
            L.wqkv8 = take((size_t)3 * EVA_D * EVA_D);
            L.wo8 = take((size_t)EVA_D * EVA_D);
        } else {
            L.wqkv16 = (const uint16_t *)take((size_t)3 * EVA_D * EVA_D * 2);
            L.wo16 = (const uint16_t *)take((size_t)EVA_D * EVA_D * 2);
        }
        L.ln2w = (const float *)take(EVA_D * 4);
        L.ln2b = (const float *)take(EVA_D * 4);
        if (v3) {
            L.w128 = take((size_t)2 * V2_HIDP * EVA_D);
            L.rs0 = (const float *)take(V2_HIDP * 4);
            L.w28 = take((size_t)EVA_D * V2_HIDP);
            L.cn0 = (const float *)take(EVA_D * 4);
            L.dn0 = (const float *)take(EVA_D * 4);
        } else {
            L.w1216 = (const uint16_t *)take((size_t)2 * V2_HIDP * EVA_D * 2);
            L.mlnw = (const float *)take(V2_HIDP * 4);
            L.mlnb = (const float *)take(V2_HIDP * 4);
            L.w216 = (const uint16_t *)take((size_t)EVA_D * V2_HIDP * 2);
        }
        L.end = off;
    }
    E->fnw = (const float *)take(EVA_D * 4);
    E->fnb = (const float *)take(EVA_D * 4);
    E->hw0 = (const uint16_t *)take((size_t)ntp * EVA_D * 2);
    E->hb0 = (const float *)take((size_t)ntp * 4);
    if (off != E->wbytes) {
        fprintf(stderr, "eva: weight layout mismatch (%zu vs %zu bytes)\n", off, E->wbytes);
        return -1;
    }
    return 0;
}

static const char *const ev_opname[EVA_PROF_OPS] = {"patch+embed", "ln1", "qkv", "flash", "oproj",
                                                     "ln2", "fc1", "fc2", "pool+head"};

// eva_profile's mark after an op of kind id (only while a profile runs, never inside the captured graph)
static int ev_mark(eva_impl *E, int id)
{
    if (!E->pon) return 0;
    if (E->pk >= (int)(sizeof(E->pev) / sizeof(E->pev[0]))) return xt_fail("eva_profile", "too many ops");
    E->pid[E->pk] = (uint8_t)id;
    XT_HIP(hipEventRecord(E->pev[E->pk++], E->st));
    return 0;
}
#define EV_OP(call, id)                                                \
    do {                                                               \
        if ((call) || ev_mark(E, (id))) return -1;                     \
    } while (0)

// The whole forward for nb inputs on stream fst (captured once per lane into lgraph[lane]), eva.h:227-310.
static int ev_forward(eva *e, hipStream_t fst)
{
    eva_impl *E = e->impl;
    void *st = (void *)fst;
    const int M = (int)E->cM, lds = (int)E->cMp, nb = (int)E->cnb;

    EV_OP(eva_k_pe(E->in, E->pe, E->pos, E->x, nb, st), 0);
    for (int i = 0; i < EVA_NL; i++) {
        const Layer &L = E->L[i];
        const bool sp = E->flags & EVA_SPARSE24;
        EV_OP(eva_k_ln(E->x, L.ln1w, L.ln1b, E->h8, E->sh, M, lds, st), 1);
        if (sp) EV_OP(eva_k_qkv_sp(E->h8, E->sh, lds, L.vqkv, L.xqkv, L.sqkv, E->cs, E->q, E->k, E->vt, M, st), 2);
        else EV_OP(eva_k_qkv(E->h8, E->sh, lds, L.wqkv, L.sqkv, E->cs, E->q, E->k, E->vt, M, st), 2);
        EV_OP(eva_k_flash(E->q, E->k, E->vt, E->h8, E->sh, lds, nb, NULL, st), 3);
        if (sp) EV_OP(eva_k_oproj_sp(E->h8, E->sh, lds, L.vo, L.xo, L.so, E->x, M, st), 4);
        else EV_OP(eva_k_oproj(E->h8, E->sh, lds, L.wo, L.so, E->x, M, st), 4);
        EV_OP(eva_k_ln(E->x, L.ln2w, L.ln2b, E->h8, E->sh, M, lds, st), 5);
        if (sp && L.rs) EV_OP(eva_k_fc1_rs_sp(E->h8, E->sh, lds, L.v12, L.x12, L.s12, E->m8, E->sm, E->stat, L.rs, M, st), 6);
        else if (sp) EV_OP(eva_k_fc1_sp(E->h8, E->sh, lds, L.v12, L.x12, L.s12, E->m8, E->sm, E->stat, M, st), 6);
        else if (L.rs) EV_OP(eva_k_fc1_rs(E->h8, E->sh, lds, L.w12, L.s12, E->m8, E->sm, E->stat, L.rs, M, st), 6);
        else EV_OP(eva_k_fc1(E->h8, E->sh, lds, L.w12, L.s12, E->m8, E->sm, E->stat, M, st), 6);
        if (sp) EV_OP(eva_k_fc2_sp(E->m8, E->sm, lds, L.v2, L.x2, L.s2, E->stat, L.cn, L.dn, E->x, M, st), 7);
        else EV_OP(eva_k_fc2(E->m8, E->sm, lds, L.w2, L.s2, E->stat, L.cn, L.dn, E->x, M, st), 7);
    }
    EV_CK(eva_k_pool(E->x, E->pool, nb, st));
    EV_CK(eva_k_lnh(E->pool, E->fnw, E->fnb, E->pn, E->pq, E->ps, nb, nb, st));
    EV_OP(eva_k_head(E->pq, E->ps, nb, E->hq, E->hs, (int)E->ldh, E->hb, E->out, nb, (int)e->nt, st), 8);
    return 0;
}

// pack head rows r0 .. r0 + n - 1 from the fp16 master, each row with its own 1x128 scales
static int ev_pack_head_rows(eva *e, uint32_t r0, uint32_t n)
{
    eva_impl *E = e->impl;
    return eva_k_quant_act(E->hmaster + (size_t)r0 * EVA_D, 2, EVA_D, (int)n, EVA_D, E->hq + (size_t)r0 * EVA_D, EVA_D,
                           E->hs + r0, (int)E->ldh, (void *)E->st);
}

// bring-up packing of layer i from its fp16 tensors in the blob (export_eva.py:52-119 on the GPU), on E->st
static int ev_pack_layer(eva_impl *E, int i)
{
    Layer &L = E->L[i];
    void *st = (void *)E->st;
    if (E->ver == 3) {
        // v3: the blob's E4M3 bytes with one scale per tensor (table[i][0..3]); the activations keep their own 1x128
        // scales, so fc1 packs h rs (rs = 1 / (adq s~)) and fc2's scale carries adq back: wdq3 adq3 (eva.h:418)
        const float *t = E->tab + (size_t)i * V3_NS;
        EV_CK(eva_k_prep_w8(L.wqkv8, EVA_D, 3 * EVA_D, EVA_D, 3 * EVA_D, EVA_D, 1, t[0], L.wqkv, L.sqkv, st));
        EV_CK(eva_k_prep_w8(L.wo8, EVA_D, EVA_D, EVA_D, EVA_D, EVA_D, 0, t[1], L.wo, L.so, st));
        EV_CK(eva_k_prep_w8(L.w128, EVA_D, 2 * V2_HIDP, EVA_D, 2 * EVA_HIDP, EVA_D, 0, t[2], L.w12, L.s12, st));
        EV_CK(eva_k_prep_w8(L.w28, V2_HIDP, EVA_D, EVA_HID, EVA_D, EVA_HIDP, 0, t[3] * t[7], L.w2, L.s2, st));
        XT_HIP(hipMemsetAsync(L.rs, 0, EVA_HIDP * 4, E->st));
        XT_HIP(hipMemcpyAsync(L.rs, L.rs0, V2_HIDP * 4, hipMemcpyDeviceToDevice, E->st));
        XT_HIP(hipMemcpyAsync(L.cn, L.cn0, EVA_D * 4, hipMemcpyDeviceToDevice, E->st));
        XT_HIP(hipMemcpyAsync(L.dn, L.dn0, EVA_D * 4, hipMemcpyDeviceToDevice, E->st));
    } else {
        EV_CK(eva_k_prep_w(L.wqkv16, EVA_D, 3 * EVA_D, EVA_D, 3 * EVA_D, EVA_D, 1, NULL, E->scratch, L.wqkv, L.sqkv, st));
        EV_CK(eva_k_prep_w(L.wo16, EVA_D, EVA_D, EVA_D, EVA_D, EVA_D, 0, NULL, E->scratch, L.wo, L.so, st));
        EV_CK(eva_k_prep_w(L.w1216, EVA_D, 2 * V2_HIDP, EVA_D, 2 * EVA_HIDP, EVA_D, 0, NULL, E->scratch, L.w12, L.s12, st));
        EV_CK(eva_k_prep_w(L.w216, V2_HIDP, EVA_D, EVA_HID, EVA_D, EVA_HIDP, 0, L.mlnw, E->scratch, L.w2, L.s2, st));
    }
    if (E->flags & EVA_SPARSE24) {
        // 2:4 magnitude pruning of the packed E4M3 weights (prune24.py "mag"); the fold term c below then sums the
        // pruned W~, which keeps the folded LayerNorm exact for the weights the GEMM uses
        struct { uint8_t *w; int n, k; uint8_t *v; uint32_t *x; } sw[4] = {
            {L.wqkv, 3 * EVA_D, EVA_D, L.vqkv, L.xqkv}, {L.wo, EVA_D, EVA_D, L.vo, L.xo},
            {L.w12, 2 * EVA_HIDP, EVA_D, L.v12, L.x12}, {L.w2, EVA_D, EVA_HIDP, L.v2, L.x2}};
        for (auto &t : sw) {
            EV_CK(eva_k_prune24(t.w, t.n, t.k, st));
            EV_CK(eva_k_pack24(t.w, t.n, t.k, t.v, t.x, NULL, st));
        }
    }
    if (E->ver == 3) {
        // c of the pruned W~ (the blob's c sums the dense one); d is the blob's
        if (E->flags & EVA_SPARSE24) EV_CK(eva_k_fold_c_rs(L.w2, L.s2, L.rs, L.cn, st));
    } else {
        EV_CK(eva_k_fold_cd(L.w2, L.s2, L.w216, V2_HIDP, L.mlnb, L.cn, L.dn, st));
    }
    return 0;
}

// make lane l's activations the set ev_forward works on
static void ev_use_lane(eva_impl *E, int l)
{
    const eva_impl::Acts &A = E->act[l];
    E->cnb = E->lnb[l];
    E->cM = E->cnb * EVA_T;
    E->cMp = (E->cM + 255) & ~255u;
    E->in = A.in, E->x = A.x, E->q = A.q, E->k = A.k, E->vt = A.vt, E->pn = A.pn;
    E->h8 = A.h8, E->m8 = A.m8, E->pq = A.pq;
    E->sh = A.sh, E->sm = A.sm, E->stat = A.stat, E->pool = A.pool, E->ps = A.ps, E->out = A.out;
}

static int ev_up(eva *e)
{
    eva_impl *E = e->impl;
    const uint32_t ntp = (e->nt0 + 7) & ~7u, nt = e->nt;

    XT_HIP(hipSetDevice(E->devno));
    if (xt_cu_count() <= 0) return xt_fail("eva_open", "cannot read the device's CU count");  // cached before any capture
    XT_HIP(hipStreamCreateWithFlags(&E->st, hipStreamNonBlocking));
    EV_ALLOC(E, E->blob, E->wbytes, false);
    if (ev_layout(E, ntp)) return -1;

    // packed weights: every layer is packed on the GPU (bring-up packing) as soon as its bytes are on the device, while
    // the host still reads the layers after it (eva.h:343-376, 452 stream on a thread of their own)
    EV_ALLOC(E, E->scratch, (size_t)2 * EVA_HIDP * EVA_D * 4, false);
    for (int i = 0; i < EVA_NL; i++) {
        Layer &L = E->L[i];
        EV_ALLOC(E, L.wqkv, (size_t)3 * EVA_D * EVA_D, false);
        EV_ALLOC(E, L.sqkv, 24 * 8 * 4, false);
        EV_ALLOC(E, L.wo, (size_t)EVA_D * EVA_D, false);
        EV_ALLOC(E, L.so, 8 * 8 * 4, false);
        EV_ALLOC(E, L.w12, (size_t)2 * EVA_HIDP * EVA_D, false);
        EV_ALLOC(E, L.s12, 44 * 8 * 4, false);
        EV_ALLOC(E, L.w2, (size_t)EVA_D * EVA_HIDP, false);
        EV_ALLOC(E, L.s2, 8 * 22 * 4, false);
        EV_ALLOC(E, L.cn, EVA_D * 4, false);
        EV_ALLOC(E, L.dn, EVA_D * 4, false);
        if (E->ver == 3) EV_ALLOC(E, L.rs, EVA_HIDP * 4, false);
        if (E->flags & EVA_SPARSE24) {
            EV_ALLOC(E, L.vqkv, (size_t)3 * EVA_D * EVA_D / 2, false);
            EV_ALLOC(E, L.xqkv, (size_t)3 * EVA_D * EVA_D / 8, false);
            EV_ALLOC(E, L.vo, (size_t)EVA_D * EVA_D / 2, false);
            EV_ALLOC(E, L.xo, (size_t)EVA_D * EVA_D / 8, false);
            EV_ALLOC(E, L.v12, (size_t)2 * EVA_HIDP * EVA_D / 2, false);
            EV_ALLOC(E, L.x12, (size_t)2 * EVA_HIDP * EVA_D / 8, false);
            EV_ALLOC(E, L.v2, (size_t)EVA_D * EVA_HIDP / 2, false);
            EV_ALLOC(E, L.x2, (size_t)EVA_D * EVA_HIDP / 8, false);
        }
    }
    int packed = 0;
    auto pack_ready = [&](size_t bytes) -> int {
        for (; packed < EVA_NL && E->L[packed].end <= bytes; packed++)
            if (ev_pack_layer(E, packed)) return -1;
        return 0;
    };
    if (xt_stream_file(E->path, 256, E->blob, E->wbytes, E->st, pack_ready) || packed != EVA_NL) {
        fprintf(stderr, "eva: cannot stream weights from %s\n", E->path);
        return -1;
    }
    // head: fp16 master (file rows, then zero extra rows with bias -16), every row packed with its own scales
    E->ldh = (nt + 63) & ~63u;
    EV_ALLOC(E, E->hmaster, (size_t)nt * EVA_D * 2, true);
    EV_ALLOC(E, E->hb, (size_t)nt * 4, false);
    EV_ALLOC(E, E->hq, (size_t)nt * EVA_D, false);
    EV_ALLOC(E, E->hs, (size_t)8 * E->ldh * 4, true);
    XT_HIP(hipMemcpyAsync(E->hmaster, E->hw0, (size_t)e->nt0 * EVA_D * 2, hipMemcpyDeviceToDevice, E->st));
    XT_HIP(hipMemcpyAsync(E->hb, E->hb0, (size_t)e->nt0 * 4, hipMemcpyDeviceToDevice, E->st));
    if (nt > e->nt0) {
        std::vector<float> nb16(nt - e->nt0, EVA_HB_OFF);
        XT_HIP(hipMemcpy(E->hb + e->nt0, nb16.data(), nb16.size() * 4, hipMemcpyHostToDevice));
    }
    EV_CK(ev_pack_head_rows(e, 0, nt));
    XT_HIP(hipHostMalloc((void **)&E->hput, (size_t)EV_HPUT_SLOTS * EV_HPUT_SLOT, hipHostMallocDefault));
    for (int s = 0; s < EV_HPUT_SLOTS; s++) XT_HIP(hipEventCreateWithFlags(&E->hput_ev[s], hipEventDisableTiming));

    // inputs, head inputs and scores of the whole batch; activations per lane, for its half
    EV_ALLOC(E, E->in_all, (size_t)E->nb * EVA_IN * 2, true);
    EV_ALLOC(E, E->pn_all, (size_t)E->nb * EVA_D * 2, true);
    EV_ALLOC(E, E->out_all, (size_t)E->nb * nt * 4, true);
    for (uint32_t l = 0; l < E->nl; l++) {
        eva_impl::Acts &A = E->act[l];
        const size_t nb = E->lnb[l], Mp = (nb * EVA_T + 255) & ~(size_t)255;
        const size_t qkvb = nb * EVA_NH * 1088 * 64 * 2;
        A.in = E->in_all + (size_t)E->loff[l] * EVA_IN;
        A.pn = E->pn_all + (size_t)E->loff[l] * EVA_D;
        A.out = E->out_all + (size_t)E->loff[l] * nt;
        EV_ALLOC(E, A.x, Mp * EVA_D * 2, true);
        EV_ALLOC(E, A.h8, Mp * EVA_D, true);
        EV_ALLOC(E, A.sh, 8 * Mp * 4, true);
        EV_ALLOC(E, A.q, qkvb, true);                   // padded attention rows stay zero forever
        EV_ALLOC(E, A.k, qkvb, true);
        EV_ALLOC(E, A.vt, qkvb, true);
        EV_ALLOC(E, A.m8, Mp * EVA_HIDP, true);
        EV_ALLOC(E, A.sm, 22 * Mp * 4, true);
        EV_ALLOC(E, A.stat, 22 * Mp * 8, true);
        EV_ALLOC(E, A.pool, nb * EVA_D * 4, true);
        EV_ALLOC(E, A.pq, nb * EVA_D, true);
        EV_ALLOC(E, A.ps, 8 * nb * 4, true);
    }
    E->lst[0] = E->st;
    XT_HIP(hipEventCreateWithFlags(&E->head_ev, hipEventDisableTiming));
    XT_HIP(hipEventRecord(E->head_ev, E->st));
    if (E->nl > 1) {
        XT_HIP(hipStreamCreateWithFlags(&E->lst[1], hipStreamNonBlocking));
        XT_HIP(hipEventCreateWithFlags(&E->lane_ev, hipEventDisableTiming));
        XT_HIP(hipEventRecord(E->lane_ev, E->lst[1]));
    }
    for (int s = 0; s < EVA_NBUF; s++) {
        XT_HIP(hipHostMalloc((void **)&e->hout[s], (size_t)E->nb * nt * 4, hipHostMallocDefault));
        if (nt > e->nt0) XT_HIP(hipHostMalloc((void **)&e->hpn[s], (size_t)E->nb * EVA_D * 2, hipHostMallocDefault));
        XT_HIP(hipEventCreateWithFlags(&E->done[s], hipEventDisableTiming));
    }
    XT_HIP(hipStreamSynchronize(E->st));

    // graph capture of the forward, once per lane (lane 1 first, so lane 0's activations stay the current set)
    for (int l = (int)E->nl - 1; l >= 0; l--) {
        ev_use_lane(E, l);
        hipGraph_t g;
        XT_HIP(hipStreamBeginCapture(E->lst[l], hipStreamCaptureModeThreadLocal));
        if (ev_forward(e, E->lst[l])) {
            (void)hipStreamEndCapture(E->lst[l], &g);
            return -1;
        }
        XT_HIP(hipStreamEndCapture(E->lst[l], &g));
        XT_HIP(hipGraphInstantiate(&E->lgraph[l], g, NULL, NULL, 0));
        XT_HIP(hipGraphDestroy(g));
        XT_HIP(hipGraphUpload(E->lgraph[l], E->lst[l]));
        XT_HIP(hipStreamSynchronize(E->lst[l]));
    }
    E->graph = E->lgraph[0];
    return 0;
}

static void *ev_boot(void *arg)
{
    eva *e = (eva *)arg;
    e->impl->bstatus = ev_up(e);
    return NULL;
}

extern "C" int eva_open_ex(eva *e, const char *weights, int device, void *pool, size_t poolb, uint32_t extra, uint32_t nb,
                           uint32_t flags)
{
    uint32_t hdr[4];
    FILE *f;

    (void)pool;
    (void)poolb;
    memset(e, 0, sizeof(*e));
    if (nb < 1 || nb > EVA_NBMAX) return xt_fail("eva_open", "batch must be 1..EVA_NBMAX");
    f = fopen(weights, "rb");
    if (!f || fread(hdr, 4, 4, f) != 4 || memcmp(hdr, "EVA2", 4) || (hdr[1] != 2 && hdr[1] != 3)) {
        fprintf(stderr, "eva: %s is not an eva02.bin v2 or v3 (export_eva.py)\n", weights);
        if (f) fclose(f);
        return -1;
    }
    float tab[EVA_NL * V3_NS];
    if (hdr[1] == 3) {  // the scale table leads the blob (eva.h:386); its host copy gives the per-tensor scales
        if (fseek(f, 256, SEEK_SET) || fread(tab, 4, EVA_NL * V3_NS, f) != EVA_NL * V3_NS) {
            fprintf(stderr, "eva: %s: truncated v3 scale table\n", weights);
            fclose(f);
            return -1;
        }
        for (int j = 0; j < EVA_NL; j++)
            for (int c = 0; c < 8; c++)
                if (!(tab[j * V3_NS + c] > 0.f) || !(tab[j * V3_NS + c] < 3e38f)) {
                    fprintf(stderr, "eva: %s: v3 scale table entry [%d][%d] is not a positive finite scale\n", weights,
                            j, c);
                    fclose(f);
                    return -1;
                }
    }
    fclose(f);
    eva_impl *E = new eva_impl();
    E->ver = hdr[1];
    if (E->ver == 3) memcpy(E->tab, tab, sizeof(tab));
    e->impl = E;
    E->path = strdup(weights);
    if (!E->path) return xt_fail("eva_open", "out of memory");
    E->devno = device;
    E->flags = flags;
    E->wbytes = hdr[3];
    E->nb = nb;
    E->nl = nb > 1 ? 2 : 1;
    E->lnb[0] = (nb + 1) / 2;
    E->lnb[1] = nb / 2;
    E->loff[0] = 0;
    E->loff[1] = E->lnb[0];
    e->nt0 = hdr[2];
    e->nt = hdr[2] + extra;
    e->ntp = (hdr[2] + 7) & ~7u;
    e->nb = nb;
    E->bstatus = -1;
    if (pthread_create(&E->boot, NULL, ev_boot, e)) return xt_fail("eva_open", "cannot start the bring-up thread");
    E->booted = 1;
    return 0;
}

extern "C" int eva_open_nb(eva *e, const char *weights, int device, void *pool, size_t poolb, uint32_t extra, uint32_t nb)
{
    return eva_open_ex(e, weights, device, pool, poolb, extra, nb, 0);
}

extern "C" int eva_open(eva *e, const char *weights, int device, void *pool, size_t poolb, uint32_t extra)
{
    return eva_open_nb(e, weights, device, pool, poolb, extra, EVA_NB);
}

extern "C" int eva_ready(eva *e)
{
    eva_impl *E = e->impl;
    if (!E) return -1;
    if (E->up) return 0;
    if (E->booted) {
        pthread_join(E->boot, NULL);
        E->booted = 0;
    }
    if (E->bstatus) return -1;
    XT_HIP(hipSetDevice(E->devno));
    E->up = 1;
    return 0;
}

extern "C" int eva_poll(eva *e)
{
    eva_impl *E = e->impl;
    if (!E) return 0;
    if (E->up) return 1;
    return E->booted ? pthread_tryjoin_np(E->boot, NULL) == 0 ? (E->booted = 0, 1) : 0 : 1;
}

extern "C" int eva_submit(eva *e, uint32_t buf, uint16_t *const *in, uint32_t n)
{
    if (eva_ready(e)) return -1;
    eva_impl *E = e->impl;
    if (buf >= EVA_NBUF || n > E->nb) return xt_fail("eva_submit", "buf >= EVA_NBUF or n > nb");
    // Every buf stages its inputs in a pinned slot of its own (this platform cannot page-lock the caller's memory in
    // place, eva.h:522). Before refilling it, only the previous batch of the same buf must be done (its input copy
    // has then left the slot): batches on the other bufs stay queued on the GPU (eva.h:627-641).
    if (!E->stage[buf]) XT_HIP(hipHostMalloc((void **)&E->stage[buf], (size_t)E->nb * EVA_IN * 2, hipHostMallocDefault));
    else XT_HIP(hipEventSynchronize(E->done[buf]));
    xt_stage_inputs(E->stage[buf], in, n, EVA_IN);
    // the first ceil(nb / 2) inputs on lane 0 (the engine stream, where head updates are ordered too), the rest on
    // lane 1 after every head update submitted before; the batch is done when lane 0 has also waited for lane 1
    const uint32_t n0 = n < E->lnb[0] ? n : E->lnb[0], n1 = n - n0;
    if (n0) XT_HIP(hipMemcpyAsync(E->in_all, E->stage[buf], (size_t)n0 * EVA_IN * 2, hipMemcpyHostToDevice, E->st));
    XT_HIP(hipGraphLaunch(E->lgraph[0], E->st));
    if (n0) XT_HIP(hipMemcpyAsync(e->hout[buf], E->out_all, (size_t)n0 * e->nt * 4, hipMemcpyDeviceToHost, E->st));
    if (e->hpn[buf] && n0) XT_HIP(hipMemcpyAsync(e->hpn[buf], E->pn_all, (size_t)n0 * EVA_D * 2, hipMemcpyDeviceToHost, E->st));
    if (n1) {
        const hipStream_t s = E->lst[1];
        const size_t o = E->loff[1];
        XT_HIP(hipStreamWaitEvent(s, E->head_ev, 0));
        XT_HIP(hipMemcpyAsync(E->in_all + o * EVA_IN, E->stage[buf] + (size_t)n0 * EVA_IN, (size_t)n1 * EVA_IN * 2,
                              hipMemcpyHostToDevice, s));
        XT_HIP(hipGraphLaunch(E->lgraph[1], s));
        XT_HIP(hipMemcpyAsync(e->hout[buf] + (size_t)n0 * e->nt, E->out_all + o * e->nt, (size_t)n1 * e->nt * 4,
                              hipMemcpyDeviceToHost, s));
        if (e->hpn[buf])
            XT_HIP(hipMemcpyAsync(e->hpn[buf] + (size_t)n0 * EVA_D, E->pn_all + o * EVA_D, (size_t)n1 * EVA_D * 2,
                                  hipMemcpyDeviceToHost, s));
        XT_HIP(hipEventRecord(E->lane_ev, s));
        XT_HIP(hipStreamWaitEvent(E->st, E->lane_ev, 0));
    }
    XT_HIP(hipEventRecord(E->done[buf], E->st));
    return 0;
}

extern "C" int eva_query(eva *e, uint32_t buf)
{
    eva_impl *E = e->impl;
    if (!E || !E->up || buf >= EVA_NBUF) return 1;
    return hipEventQuery(E->done[buf]) != hipErrorNotReady;
}

extern "C" const float *eva_wait(eva *e, uint32_t buf)
{
    eva_impl *E = e->impl;
    if (!E || !E->up || buf >= EVA_NBUF) return NULL;
    return hipEventSynchronize(E->done[buf]) == hipSuccess ? e->hout[buf] : NULL;
}

extern "C" int eva_head_put(eva *e, uint32_t j, const uint16_t *w, float bias)
{
    if (eva_ready(e)) return -1;
    eva_impl *E = e->impl;
    if (j >= e->nt) return xt_fail("eva_head_put", "row past nt");
    // stream-ordered (eva.h:643-650): the row and bias go to a pinned slot before the call returns, so w may be reused
    // at once; copies and the row's repack follow on the engine stream, and batches submitted later see the row. A
    // call waits only when every slot still has a copy in flight.
    const uint32_t slot = E->hput_next++ % EV_HPUT_SLOTS;
    XT_HIP(hipEventSynchronize(E->hput_ev[slot]));
    uint8_t *p = E->hput + (size_t)slot * EV_HPUT_SLOT;
    memcpy(p, w, EVA_D * 2);
    memcpy(p + EVA_D * 2, &bias, 4);
    // the engine stream has waited for lane 1's half of every batch submitted before, so the update follows them all;
    // lane 1's later halves wait for it (head_ev)
    XT_HIP(hipMemcpyAsync(E->hmaster + (size_t)j * EVA_D, p, EVA_D * 2, hipMemcpyHostToDevice, E->st));
    XT_HIP(hipMemcpyAsync(E->hb + j, p + EVA_D * 2, 4, hipMemcpyHostToDevice, E->st));
    EV_CK(ev_pack_head_rows(e, j, 1));
    XT_HIP(hipEventRecord(E->hput_ev[slot], E->st));
    XT_HIP(hipEventRecord(E->head_ev, E->st));
    return 0;
}

extern "C" int eva_head_get(eva *e, uint16_t *w, float *bias)
{
    if (eva_ready(e)) return -1;
    eva_impl *E = e->impl;
    XT_HIP(hipStreamSynchronize(E->st));
    XT_HIP(hipMemcpy(w, E->hw0, (size_t)e->nt0 * EVA_D * 2, hipMemcpyDeviceToHost));
    XT_HIP(hipMemcpy(bias, E->hb0, (size_t)e->nt0 * 4, hipMemcpyDeviceToHost));
    return 0;
}

extern "C" void eva_close(eva *e)
{
    eva_impl *E = e->impl;
    if (!E) return;
    if (E->booted) {
        pthread_join(E->boot, NULL);
        E->booted = 0;
    }
    (void)hipSetDevice(E->devno);
    if (E->st) (void)hipStreamSynchronize(E->st);
    if (E->lst[1]) (void)hipStreamSynchronize(E->lst[1]);
    for (int l = 0; l < 2; l++)
        if (E->lgraph[l]) (void)hipGraphExecDestroy(E->lgraph[l]);
    if (E->lst[1]) (void)hipStreamDestroy(E->lst[1]);
    if (E->lane_ev) (void)hipEventDestroy(E->lane_ev);
    if (E->head_ev) (void)hipEventDestroy(E->head_ev);
    for (int s = 0; s < EVA_NBUF; s++) {
        if (E->done[s]) (void)hipEventDestroy(E->done[s]);
        if (e->hout[s]) (void)hipHostFree(e->hout[s]);
        if (e->hpn[s]) (void)hipHostFree(e->hpn[s]);
    }
    for (int s = 0; s < EVA_NBUF; s++)
        if (E->stage[s]) (void)hipHostFree(E->stage[s]);
    if (E->hput) (void)hipHostFree(E->hput);
    for (int s = 0; s < EV_HPUT_SLOTS; s++)
        if (E->hput_ev[s]) (void)hipEventDestroy(E->hput_ev[s]);
    for (int i = 0; i < 512; i++)
        if (E->pev[i]) (void)hipEventDestroy(E->pev[i]);
    for (void *p : E->allocs) (void)hipFree(p);
    if (E->st) (void)hipStreamDestroy(E->st);
    free(E->path);
    delete E;
    memset(e, 0, sizeof(*e));
}

// eva.h:312-338: two warm direct forwards, then one with an event after every op; per op kind the GPU time between
// the previous op's event and its own, summed over the layers, printed to stderr and returned in ms[EVA_PROF_OPS]
// (when not NULL). The forward reads the device input buffer as it stands (eva_dev_input / the last submit).
extern "C" int eva_profile(eva *e, double *ms)
{
    if (eva_ready(e)) return -1;
    eva_impl *E = e->impl;
    double acc[EVA_PROF_OPS] = {0}, tot = 0;
    XT_HIP(hipStreamSynchronize(E->st));
    if (!E->pev[0])
        for (int i = 0; i < 512; i++) XT_HIP(hipEventCreate(&E->pev[i]));
    // the two halves of the batch one after the other on the engine stream, each forward twice to warm up
    auto halves = [&]() -> int {
        int rc = 0;
        for (uint32_t l = 0; l < E->nl && !rc; l++) {
            ev_use_lane(E, (int)l);
            rc = ev_forward(e, E->st);
        }
        ev_use_lane(E, 0);
        return rc;
    };
    if (halves() || halves()) return -1;
    E->pon = 1;
    E->pk = 1;
    E->pid[0] = 255;
    const hipError_t r0 = hipEventRecord(E->pev[0], E->st);
    const int rc = r0 != hipSuccess ? xt_fail("eva_profile", "hipEventRecord failed") : halves();
    E->pon = 0;
    if (rc) return -1;
    XT_HIP(hipStreamSynchronize(E->st));
    for (int i = 1; i < E->pk; i++) {
        float dt = 0.f;
        XT_HIP(hipEventElapsedTime(&dt, E->pev[i - 1], E->pev[i]));
        acc[E->pid[i]] += dt;
        tot += dt;
    }
    for (int i = 0; i < EVA_PROF_OPS; i++) {
        fprintf(stderr, "prof gpu %-12s %8.3f ms  %5.1f%%\n", ev_opname[i], acc[i], 100 * acc[i] / tot);
        if (ms) ms[i] = acc[i];
    }
    fprintf(stderr, "prof gpu batch of %u     %8.3f ms (direct launches)\n", E->nb, tot);
    return 0;
}

extern "C" const char *eva_profile_opname(int i) { return i >= 0 && i < EVA_PROF_OPS ? ev_opname[i] : NULL; }

extern "C" void *eva_dev_input(eva *e) { return eva_ready(e) ? NULL : (void *)e->impl->in_all; }
extern "C" const float *eva_dev_output(eva *e) { return eva_ready(e) ? NULL : e->impl->out_all; }
extern "C" void *eva_stream_handle(eva *e) { return eva_ready(e) ? NULL : (void *)e->impl->st; }
extern "C" int eva_run(eva *e)
{
    if (eva_ready(e)) return -1;
    eva_impl *E = e->impl;
    XT_HIP(hipGraphLaunch(E->lgraph[0], E->st));
    if (E->nl > 1) {
        XT_HIP(hipStreamWaitEvent(E->lst[1], E->head_ev, 0));
        XT_HIP(hipGraphLaunch(E->lgraph[1], E->lst[1]));
        XT_HIP(hipEventRecord(E->lane_ev, E->lst[1]));
        XT_HIP(hipStreamWaitEvent(E->st, E->lane_ev, 0));
    }
    return 0;
}
extern "C" int eva_sync(eva *e)
{
    if (eva_ready(e)) return -1;
    XT_HIP(hipStreamSynchronize(e->impl->st));
    if (e->impl->nl > 1) XT_HIP(hipStreamSynchronize(e->impl->lst[1]));
    return 0;
}
