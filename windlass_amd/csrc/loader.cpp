// loader.cpp — checkpoint tensors into a context: the MoE fields of one
// layer (wl_load_layer), routed experts into slot-pool slots
// (wl_load_experts), and packed expert files for the file tier
// (wl_st_pack_layer). Reference: glm::load_layer's MoE part and its upload
// helpers (src/glm_loader.cuh:488-620); the packed block format of
// tools/repack_experts_glm.py:5-14,46-55.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <unistd.h>

#include <cerrno>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/windlass_moe.h"
#include "host_internal.h"
#include "internal.h"
#include "safetensors.h"

namespace {

std::string fmt(const char* f, ...) __attribute__((format(printf, 1, 2)));
std::string fmt(const char* f, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, f);
    vsnprintf(buf, sizeof(buf), f, ap);
    va_end(ap);
    return buf;
}

struct Issue {
    wl_status st = WL_OK;
    std::string msg;
    bool bad() const { return st != WL_OK; }
};

// One tensor the loader expects: its name, dtype and shape ([rows, cols]
// or [n]); the reference checks dtype and byte count (upload_raw,
// src/glm_loader.cuh:498-519), this checks the shape too, so a transposed
// tensor of the right size is refused.
Issue expect(const wl_st* st, const std::string& name, const char* dtype, std::vector<uint64_t> shape,
             const wl_st::Tensor** out) {
    Issue is;
    const wl_st::Tensor* t = st->find(name);
    if (!t) {
        is.st = WL_ERR_NOT_FOUND;
        is.msg = "missing tensor " + name;
        return is;
    }
    if (t->dtype != dtype) {
        is.st = WL_ERR_FORMAT;
        is.msg = fmt("%s has dtype %s, expected %s", name.c_str(), t->dtype.c_str(), dtype);
        return is;
    }
    if (t->shape != shape) {
        std::string got, want;
        for (uint64_t d : t->shape) got += (got.empty() ? "" : ",") + std::to_string(d);
        for (uint64_t d : shape) want += (want.empty() ? "" : ",") + std::to_string(d);
        is.st = WL_ERR_FORMAT;
        is.msg = fmt("%s has shape [%s], expected [%s]", name.c_str(), got.c_str(), want.c_str());
        return is;
    }
    *out = t;
    return is;
}

// The tensors of one MXFP4 projection: weight U8 [rows, cols/2] and its
// "_scale" U8 [rows, cols/32].
Issue expect_mxfp4(const wl_st* st, const std::string& name, uint64_t rows, uint64_t cols, const wl_st::Tensor** w,
                   const wl_st::Tensor** s) {
    if (!st->find(name + "_scale")) {
        Issue is;
        is.st = st->find(name) ? WL_ERR_FORMAT : WL_ERR_NOT_FOUND;
        is.msg = st->find(name) ? name + " has no _scale: expected MXFP4" : "missing tensor " + name;
        return is;
    }
    Issue is = expect(st, name, "U8", {rows, cols / 2}, w);
    if (is.bad()) return is;
    return expect(st, name + "_scale", "U8", {rows, cols / 32}, s);
}

// The six tensors of routed expert e of checkpoint layer n, in
// wl_expert_layout order (gate_w, gate_s, up_w, up_s, down_w, down_s).
Issue expert_parts(const wl_st* st, uint32_t n, uint32_t e, uint64_t H, uint64_t I, const wl_st::Tensor** parts,
                   std::string* names) {
    const std::string P = "model.layers." + std::to_string(n) + ".mlp.experts." + std::to_string(e) + ".";
    const char* proj[3] = {"gate_proj", "up_proj", "down_proj"};
    for (int j = 0; j < 3; j++) {
        const std::string nm = P + proj[j] + ".weight";
        Issue is = expect_mxfp4(st, nm, j < 2 ? I : H, j < 2 ? H : I, &parts[2 * j], &parts[2 * j + 1]);
        if (is.bad()) return is;
        names[2 * j] = nm;
        names[2 * j + 1] = nm + "_scale";
    }
    return Issue();
}

template <typename T>
wl_status upload(wl_ctx* c, const std::vector<uint8_t>& h, T** d, const char* what) {
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, h.size() ? h.size() : 16);
    if (e != hipSuccess) return wl::ctx_fail(c, WL_ERR_OOM, fmt("hipMalloc for %s: %s", what, hipGetErrorString(e)));
    e = hipMemcpy(p, h.data(), h.size(), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(p);
        return wl::ctx_fail(c, WL_ERR_HIP, fmt("upload of %s: %s", what, hipGetErrorString(e)));
    }
    *d = (T*)p;
    return WL_OK;
}

}  // namespace

extern "C" {

wl_status wl_load_layer(wl_ctx* c, wl_st* st, uint32_t ckpt_layer, uint32_t layer) {
    if (!c) return WL_ERR_INVALID;
    if (!st) return wl::ctx_fail(c, WL_ERR_INVALID, "checkpoint is null");
    const wl_moe_config& cfg = wl::ctx_config(c);
    if (layer >= cfg.n_layers)
        return wl::ctx_fail(c, WL_ERR_INVALID, fmt("layer %u >= n_layers %u", layer, cfg.n_layers));
    const uint64_t H = cfg.hidden, E = cfg.n_routed_experts, SI = wl::ctx_shared_inter(c);
    const std::string P = "model.layers." + std::to_string(ckpt_layer) + ".";

    // Every tensor is checked before anything is read or allocated.
    const wl_st::Tensor *ln = nullptr, *rw = nullptr, *rb = nullptr;
    const std::string n_ln = P + "post_attention_layernorm.weight", n_rw = P + "mlp.gate.weight",
                      n_rb = P + "mlp.gate.e_score_correction_bias";
    Issue is;
    for (const std::string* nm : {&n_ln, &n_rw})
        if (st->find(*nm + "_scale")) return wl::ctx_fail(c, WL_ERR_FORMAT, *nm + " has a _scale: expected BF16");
    if ((is = expect(st, n_ln, "BF16", {H}, &ln)).bad() || (is = expect(st, n_rw, "BF16", {E, H}, &rw)).bad() ||
        (is = expect(st, n_rb, "F32", {E}, &rb)).bad())
        return wl::ctx_fail(c, is.st, is.msg);
    const char* proj[3] = {"gate_proj", "up_proj", "down_proj"};
    const uint64_t rows[3] = {SI, SI, H}, cols[3] = {H, H, SI};
    std::string sn[3];
    int n_scaled = 0;
    for (int j = 0; j < 3; j++) {
        sn[j] = P + "mlp.shared_experts." + proj[j] + ".weight";
        n_scaled += st->find(sn[j] + "_scale") ? 1 : 0;
    }
    if (n_scaled != 0 && n_scaled != 3)
        return wl::ctx_fail(c, WL_ERR_FORMAT, P + "mlp.shared_experts: some projections have a _scale, some not");
    const bool mx = n_scaled == 3;
    const wl_st::Tensor* sp[6] = {};
    std::string spn[6];
    for (int j = 0; j < 3; j++) {
        if (mx) {
            is = expect_mxfp4(st, sn[j], rows[j], cols[j], &sp[2 * j], &sp[2 * j + 1]);
            spn[2 * j] = sn[j];
            spn[2 * j + 1] = sn[j] + "_scale";
        } else {
            is = expect(st, sn[j], "BF16", {rows[j], cols[j]}, &sp[j]);
            spn[j] = sn[j];
        }
        if (is.bad()) return wl::ctx_fail(c, is.st, is.msg);
    }

    // Read. The shared parts go into one host buffer, uploaded once.
    auto rd = [&](const wl_st::Tensor* t, const std::string& nm, uint8_t* dst) -> wl_status {
        const wl_status s = st->read(*t, 0, t->nbytes, dst, nm);
        return s == WL_OK ? WL_OK : wl::ctx_fail(c, s, st->err);
    };
    std::vector<uint8_t> h_ln(ln->nbytes), h_rw(rw->nbytes), h_rb(rb->nbytes);
    wl_status s;
    if ((s = rd(ln, n_ln, h_ln.data())) != WL_OK || (s = rd(rw, n_rw, h_rw.data())) != WL_OK ||
        (s = rd(rb, n_rb, h_rb.data())) != WL_OK)
        return s;
    const int np = mx ? 6 : 3;
    size_t off[6] = {}, total = 0;
    for (int j = 0; j < np; j++) {
        off[j] = total;
        total += (sp[j]->nbytes + 255) & ~(size_t)255;  // each part 256-byte aligned on the device
    }
    std::vector<uint8_t> h_sh(total);
    for (int j = 0; j < np; j++)
        if ((s = rd(sp[j], spn[j], h_sh.data() + off[j])) != WL_OK) return s;

    uint16_t *d_ln = nullptr, *d_rw = nullptr;
    float* d_rb = nullptr;
    uint8_t* d_sh = nullptr;
    if ((s = upload(c, h_ln, &d_ln, "the norm weight")) != WL_OK || (s = upload(c, h_rw, &d_rw, "the router")) != WL_OK ||
        (s = upload(c, h_rb, &d_rb, "the router bias")) != WL_OK || (s = upload(c, h_sh, &d_sh, "the shared expert")) != WL_OK) {
        for (void* p : {(void*)d_ln, (void*)d_rw, (void*)d_rb}) (void)hipFree(p);
        return s;
    }
    const uint8_t* parts[6] = {};
    for (int j = 0; j < np; j++) parts[j] = d_sh + off[j];
    // bf16 shared: [gate | up | down] contiguous (the three parts are each a
    // multiple of 256 bytes at any supported shape, so off[] leaves no gaps)
    s = wl::ctx_set_layer_owned(c, layer, d_rw, d_rb, d_ln, mx ? nullptr : (const uint16_t*)d_sh, mx ? parts : nullptr);
    (void)hipFree(d_sh);  // the shared expert was converted into context memory (the call synchronised)
    return s;
}

wl_status wl_load_experts(wl_ctx* c, wl_st* st, uint32_t ckpt_layer, uint32_t layer, const uint32_t* experts,
                          uint32_t n, uint32_t first_slot, void* stream) {
    if (!c) return WL_ERR_INVALID;
    if (!st) return wl::ctx_fail(c, WL_ERR_INVALID, "checkpoint is null");
    const wl_moe_config& cfg = wl::ctx_config(c);
    if (layer >= cfg.n_layers)
        return wl::ctx_fail(c, WL_ERR_INVALID, fmt("layer %u >= n_layers %u", layer, cfg.n_layers));
    if (n == 0) return WL_OK;
    const uint32_t E = cfg.n_routed_experts;
    wl_expert_layout lay;
    if (wl_expert_layout_of(&cfg, 0, &lay) != WL_OK) return wl::ctx_fail(c, WL_ERR_INVALID, "expert layout");
    const size_t part_off[6] = {lay.gw_off, lay.gs_off, lay.uw_off, lay.us_off, lay.dw_off, lay.ds_off};
    std::vector<uint8_t*> slot(n);
    for (uint32_t i = 0; i < n; i++) {
        if (first_slot + (uint64_t)i > UINT32_MAX) return wl::ctx_fail(c, WL_ERR_INVALID, "slot index overflows");
        wl_status s = wl_slot_pool_ptr(c, first_slot + i, &slot[i]);  // checks the pool and the slot range
        if (s != WL_OK) return s;
    }
    std::vector<const wl_st::Tensor*> parts((size_t)n * 6);
    std::vector<std::string> names((size_t)n * 6);
    std::vector<uint8_t> seen(E, 0);
    for (uint32_t i = 0; i < n; i++) {
        const uint32_t e = experts ? experts[i] : i;
        if (e >= E) return wl::ctx_fail(c, WL_ERR_INVALID, fmt("expert %u >= n_routed_experts %u", e, E));
        if (seen[e]++) return wl::ctx_fail(c, WL_ERR_INVALID, fmt("expert %u listed twice", e));
        Issue is = expert_parts(st, ckpt_layer, e, cfg.hidden, cfg.moe_inter, &parts[(size_t)i * 6], &names[(size_t)i * 6]);
        if (is.bad()) return wl::ctx_fail(c, is.st, is.msg);
    }

    hipStream_t s = (hipStream_t)stream;
    uint8_t* pin[2] = {nullptr, nullptr};
    uint8_t* stage[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    wl_status rs = WL_OK;
    bool enqueued = false;
    for (int b = 0; b < 2 && rs == WL_OK; b++) {
        hipError_t e;
        if ((e = hipHostMalloc((void**)&pin[b], lay.total, hipHostMallocDefault)) != hipSuccess) {
            pin[b] = nullptr;
            rs = wl::ctx_fail(c, WL_ERR_OOM, fmt("pinned load buffer: %s", hipGetErrorString(e)));
        } else if ((e = hipMalloc((void**)&stage[b], lay.total)) != hipSuccess) {
            stage[b] = nullptr;
            rs = wl::ctx_fail(c, WL_ERR_OOM, fmt("device load staging: %s", hipGetErrorString(e)));
        } else if ((e = hipEventCreateWithFlags(&ev[b], hipEventDisableTiming)) != hipSuccess) {
            ev[b] = nullptr;
            rs = wl::ctx_fail(c, WL_ERR_HIP, fmt("load event: %s", hipGetErrorString(e)));
        }
    }
    for (uint32_t i = 0; i < n && rs == WL_OK; i++) {
        const int b = (int)(i & 1u);
        if (i >= 2) {  // the copy out of this buffer two experts ago has finished
            hipError_t e = hipEventSynchronize(ev[b]);
            if (e != hipSuccess) {
                rs = wl::ctx_fail(c, WL_ERR_HIP, fmt("load buffer wait: %s", hipGetErrorString(e)));
                break;
            }
        }
        for (int j = 0; j < 6 && rs == WL_OK; j++) {
            const wl_st::Tensor* t = parts[(size_t)i * 6 + j];
            const wl_status r = st->read(*t, 0, t->nbytes, pin[b] + part_off[j], names[(size_t)i * 6 + j]);
            if (r != WL_OK) rs = wl::ctx_fail(c, r, st->err);
        }
        if (rs != WL_OK) break;
        hipError_t e = hipMemcpyAsync(stage[b], pin[b], lay.total, hipMemcpyHostToDevice, s);
        enqueued = true;
        if (e != hipSuccess) {
            rs = wl::ctx_fail(c, WL_ERR_HIP, fmt("expert upload: %s", hipGetErrorString(e)));
            break;
        }
        if (wl::launch_expert_to_native(stage[b], slot[i], cfg.hidden, cfg.moe_inter, 0u, s) != 0) {
            rs = wl::ctx_fail(c, WL_ERR_HIP, "native conversion launch failed");
            break;
        }
        if ((e = hipEventRecord(ev[b], s)) != hipSuccess)
            rs = wl::ctx_fail(c, WL_ERR_HIP, fmt("load event record: %s", hipGetErrorString(e)));
    }
    if (enqueued) {
        hipError_t e = hipStreamSynchronize(s);
        if (e != hipSuccess && rs == WL_OK) rs = wl::ctx_fail(c, WL_ERR_HIP, fmt("load: %s", hipGetErrorString(e)));
    }
    for (int b = 0; b < 2; b++) {
        if (pin[b]) (void)hipHostFree(pin[b]);
        if (stage[b]) (void)hipFree(stage[b]);
        if (ev[b]) (void)hipEventDestroy(ev[b]);
    }
    for (uint32_t i = 0; i < n && rs == WL_OK; i++) rs = wl_slot_bind(c, layer, experts ? experts[i] : i, slot[i]);
    return rs;
}

wl_status wl_st_pack_layer(wl_st* st, const wl_moe_config* cfg, uint32_t ckpt_layer, const char* path) {
    if (!st) return WL_ERR_INVALID;
    if (!cfg || !path) {
        st->err = "config and path are required";
        return WL_ERR_INVALID;
    }
    wl_expert_layout lay;
    if (wl_expert_layout_of(cfg, 0, &lay) != WL_OK) {
        st->err = "unsupported expert shape";
        return WL_ERR_INVALID;
    }
    const uint32_t E = cfg->n_routed_experts;
    const size_t part_off[6] = {lay.gw_off, lay.gs_off, lay.uw_off, lay.us_off, lay.dw_off, lay.ds_off};
    std::vector<const wl_st::Tensor*> parts((size_t)E * 6);
    std::vector<std::string> names((size_t)E * 6);
    for (uint32_t e = 0; e < E; e++) {
        Issue is = expert_parts(st, ckpt_layer, e, cfg->hidden, cfg->moe_inter, &parts[(size_t)e * 6], &names[(size_t)e * 6]);
        if (is.bad()) {
            st->err = is.msg;
            return is.st;
        }
    }
    const int fd = ::open(path, O_WRONLY | O_CREAT | O_TRUNC, 0644);
    if (fd < 0) {
        st->err = fmt("cannot create %s: %s", path, strerror(errno));
        return WL_ERR_IO;
    }
    std::vector<uint8_t> rec(lay.total);
    wl_status rs = WL_OK;
    for (uint32_t e = 0; e < E && rs == WL_OK; e++) {
        for (int j = 0; j < 6 && rs == WL_OK; j++) {
            const wl_st::Tensor* t = parts[(size_t)e * 6 + j];
            rs = st->read(*t, 0, t->nbytes, rec.data() + part_off[j], names[(size_t)e * 6 + j]);
        }
        size_t done = 0;
        while (rs == WL_OK && done < rec.size()) {
            const ssize_t w = ::pwrite(fd, rec.data() + done, rec.size() - done, (off_t)((uint64_t)e * lay.total + done));
            if (w < 0 && errno == EINTR) continue;
            if (w <= 0) {
                st->err = fmt("write of %s: %s", path, w < 0 ? strerror(errno) : "no progress");
                rs = WL_ERR_IO;
                break;
            }
            done += (size_t)w;
        }
    }
    if (::close(fd) != 0 && rs == WL_OK) {
        st->err = fmt("close of %s: %s", path, strerror(errno));
        rs = WL_ERR_IO;
    }
    if (rs != WL_OK) (void)::unlink(path);
    return rs;
}

}  // extern "C"
