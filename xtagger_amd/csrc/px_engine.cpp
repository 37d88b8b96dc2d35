// px_engine.cpp - the PixAI tagger (ViTDet-L, 1008^2 inputs) engine behind the reference's px.h host API
// (src/engine/px.h:110-494), on HIP for one MI355X, with the same lifecycle as the wd engine: px_open returns at once;
// the bring-up (device, weights, packing, buffers, graph capture) runs on its own thread and px_ready joins it. One
// forward = one replay of a HIP graph captured once for nb inputs: patch embedding + pre-LN, 32 blocks (global
// attention in blocks 7, 15, 23, 31, px.h:38), the attention-pool head and the tag head (px.h:110-190). As in the wd
// engine, a batch runs as two halves at once (inputs 0 .. nb / 2 - 1 on the engine stream, the rest on a second lane
// with its own activations, stream and graph), each filling the CUs the other's short last rounds of tiles leave idle.
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

#define PX_PW 576             // attention-pool statistics window of px_k_hstat
#define PX_QW 288             // attention-pool pooling window of px_k_hpool / px_k_hproj
#define PX_NS 12              // v3 scale table columns per block: wdq x4, adq x4, q, k, v, pad (px.h:204, 226-238)

struct PxLayer {
    const float *ln1w, *ln1b, *bqkv, *bo, *ln2w, *ln2b, *b1, *rs, *b2;  // in the blob
    const uint16_t *wqkv16, *wo16, *w116, *w216;                        // v2: fp16 block weights in the blob
    const uint8_t *wqkv8, *wo8, *w18, *w28;                             // v3: E4M3 weights, one scale per tensor
    uint8_t *wqkv, *wo, *w1, *w2;                                       // packed E4M3
    float *sqkv, *so, *s1, *s2;
    const float *rs_fc1;                                                // rs, or NULL where the file's rs are all 1
    size_t end;                                                         // blob offset past the layer's last tensor
};

struct px_impl {
    int devno, bstatus, up, booted;
    pthread_t boot;
    char *path;
    size_t wbytes;
    uint32_t ver;                                       // blob version: 2 (fp16 weights) or 3 (E4M3 + scale table)
    float tab[PX_NL * PX_NS];                           // v3 scale table (host copy)
    uint32_t nb;                                        // inputs per launch (even)
    uint32_t nl, lnb[2], loff[2];                       // lanes in use; inputs per lane (even); first input of a lane
    uint32_t cnb, cM;                                   // inputs and token rows of the lane px_forward works on
    hipStream_t st;
    uint8_t *blob;
    const uint16_t *pe, *hpos, *wv, *hw16;
    const float *pos, *lnpw, *lnpb, *csw, *csg, *hnw, *hnb, *U, *hb;
    PxLayer L[PX_NL];
    uint8_t *hq;                                        // head E4M3 [nt][1024], each row with its own scales
    float *hs;                                          // 1x128 scale planes [8][ldh]
    uint32_t ldh;                                       // nt rounded up to 64
    float *scratch;
    // activations of the lane px_forward works on (lane 0 outside graph capture)
    uint16_t *in, *x, *q, *k, *vt, *y;
    uint8_t *h8, *o8, *m8, *oq;
    float *sh, *so8, *sm, *s, *stat, *part, *o, *oqs, *out;
    hipGraphExec_t graph;
    // two lanes, each with its own activations, stream and graph: a batch's first lnb[0] inputs run on lane 0 (st),
    // the rest on lane 1 at the same time
    struct Acts {
        uint16_t *in, *x, *q, *k, *vt, *y;
        uint8_t *h8, *o8, *m8, *oq;
        float *sh, *so8, *sm, *s, *stat, *part, *o, *oqs, *out;
    } act[2];
    uint16_t *in_all;                                   // inputs [nb][5184][592]
    float *out_all;                                     // scores [nb][nt]
    hipStream_t lst[2];
    hipGraphExec_t lgraph[2];
    hipEvent_t lane_ev;                                 // after lane 1's half of the last batch
    hipEvent_t done[PX_NBUF];
    uint16_t *stage[PX_NBUF];                           // pinned staging of each buf's inputs (at its first submit)
    std::vector<void *> allocs;
};

static int px_alloc(px_impl *E, void **p, size_t bytes, bool zero)
{
    if (hipMalloc(p, bytes ? bytes : 16) != hipSuccess) return xt_fail("hipMalloc", "out of device memory");
    E->allocs.push_back(*p);
    if (zero && hipMemset(*p, 0, bytes) != hipSuccess) return xt_fail("hipMemset", "failed");
    return 0;
}
#define PX_ALLOC(E, p, bytes, zero)                                    \
    do {                                                               \
        void *tmp_;                                                    \
        if (px_alloc((E), &tmp_, (bytes), (zero))) return -1;          \
        (p) = (decltype(p))tmp_;                                       \
    } while (0)
#define PX_CK(call)                                                    \
    do {                                                               \
        if ((call)) return -1;                                         \
    } while (0)

// Blob layout of export_pixai.py (px.h:196-253): every tensor on a 256-byte boundary; version 3 leads with the
// [32][12] scale table and holds the block weights as E4M3 bytes, version 2 as fp16.
static int px_layout(px_impl *E, uint32_t ntp)
{
    size_t off = 0;
    auto take = [&](size_t bytes) -> uint8_t * {
        off = (off + 255) & ~(size_t)255;
        uint8_t *p = E->blob + off;
        off += bytes;
        return p;
    };
    const bool v3 = E->ver == 3;
    const size_t wb = v3 ? 1 : 2;
    if (v3) take((size_t)PX_NL * PX_NS * 4);
    E->pe = (const uint16_t *)take((size_t)EVA_D * EVA_K0P * 2);
    E->pos = (const float *)take((size_t)PX_T * EVA_D * 4);
    E->lnpw = (const float *)take(EVA_D * 4);
    E->lnpb = (const float *)take(EVA_D * 4);
    E->csw = (const float *)take((size_t)PX_LW * 32 * 2 * 4);
    E->csg = (const float *)take((size_t)PX_T * 32 * 2 * 4);
    for (int i = 0; i < PX_NL; i++) {
        PxLayer &L = E->L[i];
        L.ln1w = (const float *)take(EVA_D * 4);
        L.ln1b = (const float *)take(EVA_D * 4);
        const uint8_t *wqkv = take((size_t)3 * EVA_D * EVA_D * wb);
        L.bqkv = (const float *)take(3 * EVA_D * 4);
        const uint8_t *wo = take((size_t)EVA_D * EVA_D * wb);
        L.bo = (const float *)take(EVA_D * 4);
        L.ln2w = (const float *)take(EVA_D * 4);
        L.ln2b = (const float *)take(EVA_D * 4);
        const uint8_t *w1 = take((size_t)PX_HID * EVA_D * wb);
        L.b1 = (const float *)take(PX_HID * 4);
        L.rs = (const float *)take(PX_HID * 4);
        const uint8_t *w2 = take((size_t)EVA_D * PX_HID * wb);
        L.b2 = (const float *)take(EVA_D * 4);
        if (v3) {
            L.wqkv8 = wqkv, L.wo8 = wo, L.w18 = w1, L.w28 = w2;
        } else {
            L.wqkv16 = (const uint16_t *)wqkv, L.wo16 = (const uint16_t *)wo;
            L.w116 = (const uint16_t *)w1, L.w216 = (const uint16_t *)w2;
        }
        L.end = off;
    }
    E->hnw = (const float *)take(EVA_D * 4);
    E->hnb = (const float *)take(EVA_D * 4);
    E->U = (const float *)take((size_t)16 * EVA_D * 4);
    E->hpos = (const uint16_t *)take((size_t)PX_T * EVA_D * 2);
    E->wv = (const uint16_t *)take((size_t)EVA_D * EVA_D * 2);
    E->hw16 = (const uint16_t *)take((size_t)ntp * EVA_D * 2);
    E->hb = (const float *)take((size_t)ntp * 4);
    if (off != E->wbytes) {
        fprintf(stderr, "px: weight layout mismatch (%zu vs %zu bytes)\n", off, E->wbytes);
        return -1;
    }
    return 0;
}

// make lane l's activations the set px_forward works on
static void px_use_lane(px_impl *E, int l)
{
    const px_impl::Acts &A = E->act[l];
    E->cnb = E->lnb[l];
    E->cM = E->lnb[l] * PX_T;
    E->in = A.in, E->x = A.x, E->q = A.q, E->k = A.k, E->vt = A.vt, E->y = A.y;
    E->h8 = A.h8, E->o8 = A.o8, E->m8 = A.m8, E->oq = A.oq;
    E->sh = A.sh, E->so8 = A.so8, E->sm = A.sm, E->s = A.s, E->stat = A.stat, E->part = A.part, E->o = A.o;
    E->oqs = A.oqs, E->out = A.out;
}

// The whole forward for nb inputs on stream fst (captured once per lane into lgraph[lane]), px.h:110-190.
static int px_forward(px *p, hipStream_t fst)
{
    px_impl *E = p->impl;
    void *st = (void *)fst;
    const int M = (int)E->cM, nb = (int)E->cnb;

    PX_CK(px_k_pe(E->in, E->pe, E->x, M, st));
    PX_CK(px_k_pembed(E->x, E->pos, PX_T, E->lnpw, E->lnpb, M, st));
    for (int i = 0; i < PX_NL; i++) {
        const PxLayer &L = E->L[i];
        const bool glob = (i & 7) == 7;
        const int Ls = glob ? PX_T : PX_LW;
        PX_CK(eva_k_ln(E->x, L.ln1w, L.ln1b, E->h8, E->sh, M, M, st));
        PX_CK(px_k_qkv(E->h8, E->sh, M, L.wqkv, L.sqkv, L.bqkv, glob ? E->csg : E->csw, Ls, E->q, E->k, E->vt, M, st));
        PX_CK(eva_k_flash_seq(E->q, E->k, E->vt, E->o8, E->so8, M, M / Ls, Ls, Ls, NULL, st));
        PX_CK(px_k_proj(E->o8, E->so8, M, L.wo, L.so, L.bo, E->x, M, st));
        PX_CK(eva_k_ln(E->x, L.ln2w, L.ln2b, E->h8, E->sh, M, M, st));
        PX_CK(px_k_fc1(E->h8, E->sh, M, L.w1, L.s1, L.b1, L.rs_fc1, E->m8, E->sm, M, st));
        PX_CK(px_k_fc2(E->m8, E->sm, M, L.w2, L.s2, L.b2, E->x, M, st));
    }
    PX_CK(px_k_hln(E->x, E->hnw, E->hnb, E->hpos, PX_T, E->U, E->y, E->s, M, st));
    PX_CK(px_k_hstat(E->s, E->stat, nb, PX_T, st));
    PX_CK(px_k_hpool(E->s, E->stat, E->y, nullptr, E->part, nb, PX_T, st));
    PX_CK(px_k_hproj(E->part, PX_T / PX_QW, E->wv, E->o, nb, st));
    PX_CK(eva_k_quant_act(E->o, 1, EVA_D, nb, EVA_D, E->oq, EVA_D, E->oqs, nb, st));
    PX_CK(eva_k_head(E->oq, E->oqs, nb, E->hq, E->hs, (int)E->ldh, E->hb, E->out, nb, (int)p->nt, st));
    return 0;
}

// bring-up packing of block i's GEMM weights from the blob, on E->st; q / k rows of Wqkv quad-split for the RoPE
// epilogue
static int px_pack_layer(px_impl *E, int i)
{
    PxLayer &L = E->L[i];
    void *st = (void *)E->st;
    if (E->ver == 3) {
        // v3: the blob's E4M3 bytes with one scale per tensor (table[i][0..3], px.h:234-237); the smoothing is
        // already folded into the LayerNorms, V rows and weights. The activations keep their own 1x128 scales, so
        // fc1 packs gelu(u) rs with the blob's rs = 1 / (adq3 s3) (export_pixai.py:98) and fc2's scale carries adq3
        // back: wdq3 adq3
        const float *t = E->tab + (size_t)i * PX_NS;
        PX_CK(eva_k_prep_w8(L.wqkv8, EVA_D, 3 * EVA_D, EVA_D, 3 * EVA_D, EVA_D, 1, t[0], L.wqkv, L.sqkv, st));
        PX_CK(eva_k_prep_w8(L.wo8, EVA_D, EVA_D, EVA_D, EVA_D, EVA_D, 0, t[1], L.wo, L.so, st));
        PX_CK(eva_k_prep_w8(L.w18, EVA_D, PX_HID, EVA_D, PX_HID, EVA_D, 0, t[2], L.w1, L.s1, st));
        PX_CK(eva_k_prep_w8(L.w28, PX_HID, EVA_D, PX_HID, EVA_D, PX_HID, 0, t[3] * t[7], L.w2, L.s2, st));
        return 0;
    }
    PX_CK(eva_k_prep_w(L.wqkv16, EVA_D, 3 * EVA_D, EVA_D, 3 * EVA_D, EVA_D, 1, NULL, E->scratch, L.wqkv, L.sqkv, st));
    PX_CK(eva_k_prep_w(L.wo16, EVA_D, EVA_D, EVA_D, EVA_D, EVA_D, 0, NULL, E->scratch, L.wo, L.so, st));
    PX_CK(eva_k_prep_w(L.w116, EVA_D, PX_HID, EVA_D, PX_HID, EVA_D, 0, NULL, E->scratch, L.w1, L.s1, st));
    PX_CK(eva_k_prep_w(L.w216, PX_HID, EVA_D, PX_HID, EVA_D, PX_HID, 0, NULL, E->scratch, L.w2, L.s2, st));
    return 0;
}

static int px_up(px *p)
{
    px_impl *E = p->impl;

    XT_HIP(hipSetDevice(E->devno));
    if (xt_cu_count() <= 0) return xt_fail("px_open", "cannot read the device's CU count");  // cached before any capture
    XT_HIP(hipStreamCreateWithFlags(&E->st, hipStreamNonBlocking));
    PX_ALLOC(E, E->blob, E->wbytes, false);
    if (px_layout(E, p->ntp)) return -1;

    // packed weights: each block is packed on the GPU as soon as its bytes are on the device, while the host still
    // reads the blocks after it
    PX_ALLOC(E, E->scratch, (size_t)PX_HID * EVA_D * 4, false);
    for (int i = 0; i < PX_NL; i++) {
        PxLayer &L = E->L[i];
        PX_ALLOC(E, L.wqkv, (size_t)3 * EVA_D * EVA_D, false);
        PX_ALLOC(E, L.sqkv, 24 * 8 * 4, false);
        PX_ALLOC(E, L.wo, (size_t)EVA_D * EVA_D, false);
        PX_ALLOC(E, L.so, 8 * 8 * 4, false);
        PX_ALLOC(E, L.w1, (size_t)PX_HID * EVA_D, false);
        PX_ALLOC(E, L.s1, 37 * 8 * 4, false);
        PX_ALLOC(E, L.w2, (size_t)EVA_D * PX_HID, false);
        PX_ALLOC(E, L.s2, 8 * 37 * 4, false);
    }
    int packed = 0;
    auto pack_ready = [&](size_t bytes) -> int {
        for (; packed < PX_NL && E->L[packed].end <= bytes; packed++)
            if (px_pack_layer(E, packed)) return -1;
        return 0;
    };
    if (xt_stream_file(E->path, 256, E->blob, E->wbytes, E->st, pack_ready) || packed != PX_NL) {
        fprintf(stderr, "px: cannot stream weights from %s\n", E->path);
        return -1;
    }

    // per-unit fc1 multipliers: a file without calibration holds ones (export_pixai.py:83), and multiplying by 1 is
    // exact, so fc1 then runs without the multiply; a v3 file holds 1 / (adq3 s3)
    std::vector<float> rs(PX_HID);
    for (int i = 0; i < PX_NL; i++) {
        PxLayer &L = E->L[i];
        XT_HIP(hipMemcpy(rs.data(), L.rs, PX_HID * 4, hipMemcpyDeviceToHost));
        bool ones = true;
        for (float v : rs) ones = ones && v == 1.0f;
        L.rs_fc1 = ones ? NULL : L.rs;
    }

    // head: the file's fp16 rows, each packed with its own 1x128 scales
    E->ldh = (p->nt + 63) & ~63u;
    PX_ALLOC(E, E->hq, (size_t)p->nt * EVA_D, false);
    PX_ALLOC(E, E->hs, (size_t)8 * E->ldh * 4, true);
    PX_CK(eva_k_quant_act(E->hw16, 2, EVA_D, (int)p->nt, EVA_D, E->hq, EVA_D, E->hs, (int)E->ldh, (void *)E->st));

    // inputs and scores of the whole batch; activations per lane, for its half
    PX_ALLOC(E, E->in_all, (size_t)E->nb * PX_IN * 2, true);
    PX_ALLOC(E, E->out_all, (size_t)E->nb * p->nt * 4, true);
    for (uint32_t l = 0; l < E->nl; l++) {
        px_impl::Acts &A = E->act[l];
        const size_t nb = E->lnb[l], M = nb * PX_T;
        A.in = E->in_all + (size_t)E->loff[l] * PX_IN;
        A.out = E->out_all + (size_t)E->loff[l] * p->nt;
        PX_ALLOC(E, A.x, M * EVA_D * 2, true);
        PX_ALLOC(E, A.h8, M * EVA_D, true);
        PX_ALLOC(E, A.sh, 8 * M * 4, true);
        PX_ALLOC(E, A.q, M * EVA_D * 2, true);
        PX_ALLOC(E, A.k, M * EVA_D * 2, true);
        PX_ALLOC(E, A.vt, M * EVA_D * 2, true);
        PX_ALLOC(E, A.o8, M * EVA_D, true);
        PX_ALLOC(E, A.so8, 8 * M * 4, true);
        PX_ALLOC(E, A.m8, M * PX_HID, true);
        PX_ALLOC(E, A.sm, (PX_HID / 128) * M * 4, true);
        PX_ALLOC(E, A.y, M * EVA_D * 2, true);
        PX_ALLOC(E, A.s, M * 16 * 4, true);
        PX_ALLOC(E, A.stat, nb * (PX_T / PX_PW) * 16 * 2 * 4, true);
        PX_ALLOC(E, A.part, nb * (PX_T / PX_QW) * 16 * EVA_D * 4, true);
        PX_ALLOC(E, A.o, nb * EVA_D * 4, true);
        PX_ALLOC(E, A.oq, nb * EVA_D, true);
        PX_ALLOC(E, A.oqs, 8 * nb * 4, true);
    }
    if (E->nl > 1) XT_HIP(hipStreamCreateWithFlags(&E->lst[1], hipStreamNonBlocking));
    E->lst[0] = E->st;
    XT_HIP(hipEventCreateWithFlags(&E->lane_ev, hipEventDisableTiming));
    for (int s = 0; s < PX_NBUF; s++) {
        XT_HIP(hipHostMalloc((void **)&p->hout[s], (size_t)E->nb * p->nt * 4, hipHostMallocDefault));
        XT_HIP(hipEventCreateWithFlags(&E->done[s], hipEventDisableTiming));
    }
    XT_HIP(hipStreamSynchronize(E->st));

    // one graph per lane (lane 1 first, so lane 0's activations stay the current set)
    for (int l = (int)E->nl - 1; l >= 0; l--) {
        px_use_lane(E, l);
        hipGraph_t g;
        XT_HIP(hipStreamBeginCapture(E->lst[l], hipStreamCaptureModeThreadLocal));
        if (px_forward(p, E->lst[l])) {
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

static void *px_boot(void *arg)
{
    px *p = (px *)arg;
    p->impl->bstatus = px_up(p);
    return NULL;
}

extern "C" int px_open_nb(px *p, const char *weights, int device, void *pool, size_t poolb, uint32_t nb)
{
    uint32_t hdr[4];
    FILE *f;

    (void)pool;
    (void)poolb;
    memset(p, 0, sizeof(*p));
    if (nb < 2 || nb > 100 || (nb & 1)) return xt_fail("px_open", "batch must be even, 2..100");
    f = fopen(weights, "rb");
    if (!f || fread(hdr, 4, 4, f) != 4 || memcmp(hdr, "PXAI", 4) || (hdr[1] != 2 && hdr[1] != 3) || hdr[2] == 0) {
        fprintf(stderr, "px: %s is not a pixai.bin v2 or v3 (export_pixai.py)\n", weights);
        if (f) fclose(f);
        return -1;
    }
    float tab[PX_NL * PX_NS];
    if (hdr[1] == 3) {  // the scale table leads the blob (px.h:204, 365); its host copy gives the per-tensor scales
        if (fseek(f, 256, SEEK_SET) || fread(tab, 4, PX_NL * PX_NS, f) != PX_NL * PX_NS) {
            fprintf(stderr, "px: %s: truncated v3 scale table\n", weights);
            fclose(f);
            return -1;
        }
        for (int j = 0; j < PX_NL; j++)
            for (int c = 0; c < 8; c++)
                if (!(tab[j * PX_NS + c] > 0.f) || !(tab[j * PX_NS + c] < 3e38f)) {
                    fprintf(stderr, "px: %s: v3 scale table entry [%d][%d] is not a positive finite scale\n", weights,
                            j, c);
                    fclose(f);
                    return -1;
                }
    }
    fclose(f);
    px_impl *E = new px_impl();
    E->ver = hdr[1];
    if (E->ver == 3) memcpy(E->tab, tab, sizeof(tab));
    p->impl = E;
    E->path = strdup(weights);
    if (!E->path) return xt_fail("px_open", "out of memory");
    E->devno = device;
    E->wbytes = hdr[3];
    E->nb = nb;
    // halves of even size (an odd half would leave a partial pair of images): nb = 2 runs on one lane, 6 as 4 + 2
    E->lnb[0] = ((uint32_t)nb / 2 + 1) & ~1u;
    E->lnb[1] = (uint32_t)nb - E->lnb[0];
    E->nl = E->lnb[1] ? 2 : 1;
    E->loff[0] = 0;
    E->loff[1] = E->lnb[0];
    p->nt = hdr[2];
    p->ntp = (hdr[2] + 7) & ~7u;
    p->nb = nb;
    E->bstatus = -1;
    if (pthread_create(&E->boot, NULL, px_boot, p)) return xt_fail("px_open", "cannot start the bring-up thread");
    E->booted = 1;
    return 0;
}

extern "C" int px_open(px *p, const char *weights, int device, void *pool, size_t poolb)
{
    return px_open_nb(p, weights, device, pool, poolb, PX_NB);
}

extern "C" int px_ready(px *p)
{
    px_impl *E = p->impl;
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

extern "C" int px_poll(px *p)
{
    px_impl *E = p->impl;
    if (!E) return 0;
    if (E->up) return 1;
    return E->booted ? pthread_tryjoin_np(E->boot, NULL) == 0 ? (E->booted = 0, 1) : 0 : 1;
}

extern "C" int px_submit(px *p, uint32_t buf, uint16_t *const *in, uint32_t n)
{
    if (px_ready(p)) return -1;
    px_impl *E = p->impl;
    if (buf >= PX_NBUF || n > E->nb) return xt_fail("px_submit", "buf >= PX_NBUF or n > nb");
    // a pinned staging slot per buf: refilling it waits only for the previous batch of the same buf (px.h:406-419)
    if (!E->stage[buf]) XT_HIP(hipHostMalloc((void **)&E->stage[buf], (size_t)E->nb * PX_IN * 2, hipHostMallocDefault));
    else XT_HIP(hipEventSynchronize(E->done[buf]));
    xt_stage_inputs(E->stage[buf], in, n, PX_IN);
    // the first lnb[0] inputs on the engine stream, the rest on lane 1; the batch is done when the engine stream has
    // also waited for lane 1
    const uint32_t n0 = n < E->lnb[0] ? n : E->lnb[0], n1 = n - n0;
    if (n0) XT_HIP(hipMemcpyAsync(E->in_all, E->stage[buf], (size_t)n0 * PX_IN * 2, hipMemcpyHostToDevice, E->st));
    XT_HIP(hipGraphLaunch(E->lgraph[0], E->st));
    if (n0) XT_HIP(hipMemcpyAsync(p->hout[buf], E->out_all, (size_t)n0 * p->nt * 4, hipMemcpyDeviceToHost, E->st));
    if (n1) {
        const hipStream_t s = E->lst[1];
        XT_HIP(hipMemcpyAsync(E->in_all + (size_t)E->loff[1] * PX_IN, E->stage[buf] + (size_t)n0 * PX_IN,
                              (size_t)n1 * PX_IN * 2, hipMemcpyHostToDevice, s));
        XT_HIP(hipGraphLaunch(E->lgraph[1], s));
        XT_HIP(hipMemcpyAsync(p->hout[buf] + (size_t)n0 * p->nt, E->out_all + (size_t)E->loff[1] * p->nt,
                              (size_t)n1 * p->nt * 4, hipMemcpyDeviceToHost, s));
        XT_HIP(hipEventRecord(E->lane_ev, s));
        XT_HIP(hipStreamWaitEvent(E->st, E->lane_ev, 0));
    }
    XT_HIP(hipEventRecord(E->done[buf], E->st));
    return 0;
}

extern "C" int px_query(px *p, uint32_t buf)
{
    px_impl *E = p->impl;
    if (!E || !E->up || buf >= PX_NBUF) return 1;
    return hipEventQuery(E->done[buf]) != hipErrorNotReady;
}

extern "C" const float *px_wait(px *p, uint32_t buf)
{
    px_impl *E = p->impl;
    if (!E || !E->up || buf >= PX_NBUF) return NULL;
    return hipEventSynchronize(E->done[buf]) == hipSuccess ? p->hout[buf] : NULL;
}

extern "C" void px_close(px *p)
{
    px_impl *E = p->impl;
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
    for (int s = 0; s < PX_NBUF; s++) {
        if (E->done[s]) (void)hipEventDestroy(E->done[s]);
        if (p->hout[s]) (void)hipHostFree(p->hout[s]);
    }
    for (int s = 0; s < PX_NBUF; s++)
        if (E->stage[s]) (void)hipHostFree(E->stage[s]);
    for (void *ptr : E->allocs) (void)hipFree(ptr);
    if (E->st) (void)hipStreamDestroy(E->st);
    free(E->path);
    delete E;
    memset(p, 0, sizeof(*p));
}

extern "C" void *px_dev_input(px *p) { return px_ready(p) ? NULL : (void *)p->impl->in_all; }
extern "C" const float *px_dev_output(px *p) { return px_ready(p) ? NULL : p->impl->out_all; }
extern "C" void *px_stream_handle(px *p) { return px_ready(p) ? NULL : (void *)p->impl->st; }
extern "C" int px_run(px *p)
{
    if (px_ready(p)) return -1;
    px_impl *E = p->impl;
    XT_HIP(hipGraphLaunch(E->lgraph[0], E->st));
    if (E->nl > 1) {
        XT_HIP(hipGraphLaunch(E->lgraph[1], E->lst[1]));
        XT_HIP(hipEventRecord(E->lane_ev, E->lst[1]));
        XT_HIP(hipStreamWaitEvent(E->st, E->lane_ev, 0));
    }
    return 0;
}
extern "C" int px_sync(px *p)
{
    if (px_ready(p)) return -1;
    XT_HIP(hipStreamSynchronize(p->impl->st));
    if (p->impl->lst[1]) XT_HIP(hipStreamSynchronize(p->impl->lst[1]));
    return 0;
}
