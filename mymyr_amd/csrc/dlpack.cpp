// DLPack export of device arrays (include/mymyr_amd.h, "DLPack"): reference-counted library buffers, views of them and
// of a state set's rows as DLPack 1.x managed tensors with device type kDLROCM, the producer-to-consumer stream
// handoff, and a PyCapsule destructor for Python hosts.
//
// Follows the reference's export (python/src/arrays.cpp:100-235): the view's shape and strides live in a context owned
// by the managed tensor, the byte offset is folded into the data pointer (consumers such as torch reject a nonzero
// byte_offset), and the deleter releases the owner without needing any interpreter state. The stream handoff follows
// python/src/dlpack.hpp:1-94: an event recorded on the producer's stream that the consumer's stream waits for.

#include "../../include/mymyr_amd.h"

#include "capi_internal.hpp"
#include "runtime.hpp"
#include "state_set.hpp"

#include <dlfcn.h>

#include <stdexcept>
#include <vector>

struct mya_buffer
{
    void* data = nullptr;
    uint64_t bytes = 0;
    int device = 0;
    std::atomic<int> refs{1};
};

namespace mya
{
namespace
{
void buffer_unref(mya_buffer* b)
{
    if (b->refs.fetch_sub(1, std::memory_order_acq_rel) != 1)
        return;
    int cur = 0;
    const bool switch_device = hipGetDevice(&cur) == hipSuccess && cur != b->device;
    if (switch_device)
        (void)hipSetDevice(b->device);
    dev_free(b->data);
    if (switch_device)
        (void)hipSetDevice(cur);
    delete b;
}

/// What a managed tensor owns: its shape and strides and one reference to the buffer or set behind the data.
struct Ctx
{
    std::vector<int64_t> shape, strides;
    mya_buffer* buffer = nullptr;
    mya_hashset* set = nullptr;

    void release()
    {
        if (buffer)
            buffer_unref(buffer);
        if (set)
            hashset_unref(set);
    }
};

template<class M>
void delete_managed(M* m)
{
    auto* ctx = static_cast<Ctx*>(m->manager_ctx);
    ctx->release();
    delete ctx;
    delete m;
}

void fill(mya_dl_tensor& t, void* data, int device, mya_dl_dtype dtype, Ctx* ctx)
{
    t.data = data;
    t.device = {MYA_DL_ROCM, device};
    t.ndim = static_cast<int32_t>(ctx->shape.size());
    t.dtype = dtype;
    t.shape = ctx->shape.data();
    t.strides = ctx->strides.data();
    t.byte_offset = 0;
}

/// The managed tensor (versioned or legacy) over `data`; takes ownership of ctx (released on failure).
void* make_managed(void* data, int device, mya_dl_dtype dtype, Ctx* ctx, uint64_t flags, int versioned)
{
    if (versioned)
    {
        auto* m = new mya_dl_managed_versioned{};
        m->version = {MYA_DL_MAJOR, MYA_DL_MINOR};
        m->manager_ctx = ctx;
        m->deleter = &delete_managed<mya_dl_managed_versioned>;
        m->flags = flags;
        fill(m->dl_tensor, data, device, dtype, ctx);
        return m;
    }
    if (flags)
        throw std::invalid_argument("mymyr_amd: dlpack export: flags need a versioned tensor");
    auto* m = new mya_dl_managed{};
    m->manager_ctx = ctx;
    m->deleter = &delete_managed<mya_dl_managed>;
    fill(m->dl_tensor, data, device, dtype, ctx);
    return m;
}

/// Makes later work on the consumer stream wait for the work queued so far on the producer stream.
void handoff(hipStream_t producer, int64_t consumer)
{
    if (consumer == MYA_DL_STREAM_NONE)
        return;
    if (consumer < -1)
        throw std::invalid_argument("mymyr_amd: dlpack export: invalid consumer stream");
    auto* c = reinterpret_cast<hipStream_t>(static_cast<intptr_t>(consumer));
    if (c == producer)
        return;
    hipEvent_t e = event_acquire();
    try
    {
        hip_check(hipEventRecord(e, producer), "dlpack export: event record");
        hip_check(hipStreamWaitEvent(c, e, 0), "dlpack export: stream wait");
    }
    catch (...)
    {
        event_release(e);
        throw;
    }
    event_release(e);  // the wait already holds the recorded point; a later record does not move it
}

mya_dl_dtype checked_dtype(uint8_t code, uint8_t bits)
{
    const bool ok_bits = bits == 8 || bits == 16 || bits == 32 || bits == 64;
    const bool ok = (code == MYA_DL_INT || code == MYA_DL_UINT) ? ok_bits
                    : code == MYA_DL_FLOAT                      ? bits == 16 || bits == 32 || bits == 64
                    : code == MYA_DL_BOOL                       ? bits == 8
                                                                : false;
    if (!ok)
        throw std::invalid_argument("mymyr_amd: dlpack export: unsupported dtype (code " + std::to_string(code) + ", bits " +
                                    std::to_string(bits) + ")");
    return {code, bits, 1};
}
}  // namespace

void hashset_unref(mya_hashset* h)
{
    if (h->refs.fetch_sub(1, std::memory_order_acq_rel) != 1)
        return;
    state_set_destroy(h->set);
    delete h;
}
}  // namespace mya

using namespace mya;

extern "C" {

int mya_buffer_create(uint64_t bytes, mya_buffer** out)
{
    return guarded([&] {
        if (!out)
            throw std::invalid_argument("mymyr_amd: buffer_create: null output");
        auto b = std::make_unique<mya_buffer>();
        hip_check(hipGetDevice(&b->device), "hipGetDevice");
        b->data = dev_alloc<unsigned char>(bytes, "buffer");
        b->bytes = bytes;
        *out = b.release();
    });
}

void* mya_buffer_data(const mya_buffer* buffer) { return buffer ? buffer->data : nullptr; }

uint64_t mya_buffer_bytes(const mya_buffer* buffer) { return buffer ? buffer->bytes : 0; }

void mya_buffer_release(mya_buffer* buffer)
{
    if (buffer)
        buffer_unref(buffer);
}

int mya_buffer_export(mya_buffer* buffer, uint64_t byte_offset, uint8_t code, uint8_t bits, int32_t ndim,
                      const int64_t* shape, const int64_t* strides, uint64_t flags, void* producer_stream,
                      int64_t consumer_stream, int versioned, void** out)
{
    return guarded([&] {
        if (!buffer || !out || (ndim > 0 && !shape))
            throw std::invalid_argument("mymyr_amd: buffer_export: null argument");
        if (ndim < 0 || ndim > 8)
            throw std::invalid_argument("mymyr_amd: buffer_export: ndim must be in [0, 8]");
        if (flags & ~uint64_t{MYA_DL_FLAG_READ_ONLY})
            throw std::invalid_argument("mymyr_amd: buffer_export: unknown flags");
        const mya_dl_dtype dtype = checked_dtype(code, bits);
        const uint64_t esize = bits / 8;
        if (byte_offset % esize)
            throw std::invalid_argument("mymyr_amd: buffer_export: byte_offset is not a multiple of the element size");
        auto ctx = std::make_unique<Ctx>();
        ctx->shape.assign(shape, shape + ndim);
        ctx->strides.resize(ndim);
        unsigned __int128 running = 1;  // row-major stride of dimension d
        for (int d = ndim; d-- > 0;)
        {
            if (shape[d] < 0)
                throw std::invalid_argument("mymyr_amd: buffer_export: negative extent");
            if (!strides && running > static_cast<unsigned __int128>(INT64_MAX))
                throw std::invalid_argument("mymyr_amd: buffer_export: the view reaches past the buffer");
            ctx->strides[d] = strides ? strides[d] : static_cast<int64_t>(running);
            if (ctx->strides[d] < 0)
                throw std::invalid_argument("mymyr_amd: buffer_export: negative stride");
            running *= static_cast<uint64_t>(shape[d] ? shape[d] : 1);
        }
        // the last byte touched: offset + sum (extent - 1) * stride * esize, each term checked before it is scaled
        bool empty = false, past = false;
        unsigned __int128 last = byte_offset;
        for (int d = 0; d < ndim; ++d)
        {
            if (shape[d] == 0)
            {
                empty = true;
                continue;
            }
            const unsigned __int128 span = static_cast<unsigned __int128>(shape[d] - 1) * static_cast<uint64_t>(ctx->strides[d]);
            if (span > buffer->bytes)
                past = true;
            else
                last += span * esize;
        }
        if (!empty && (past || last + esize > buffer->bytes))
            throw std::invalid_argument("mymyr_amd: buffer_export: the view reaches past the buffer's " +
                                        std::to_string(buffer->bytes) + " bytes");
        if (empty && byte_offset > buffer->bytes)
            throw std::invalid_argument("mymyr_amd: buffer_export: byte_offset past the buffer");
        handoff(static_cast<hipStream_t>(producer_stream), consumer_stream);
        buffer->refs.fetch_add(1, std::memory_order_relaxed);
        ctx->buffer = buffer;
        Ctx* c = ctx.release();
        try
        {
            *out = make_managed(static_cast<unsigned char*>(buffer->data) + byte_offset, buffer->device, dtype, c, flags,
                                versioned);
        }
        catch (...)
        {
            c->release();
            delete c;
            throw;
        }
    });
}

int mya_hashset_export_rows(mya_hashset* set, uint64_t flags, int64_t consumer_stream, int versioned, void** out)
{
    return guarded([&] {
        if (!set || !out)
            throw std::invalid_argument("mymyr_amd: hashset_export_rows: null argument");
        if (flags & ~uint64_t{MYA_DL_FLAG_READ_ONLY})
            throw std::invalid_argument("mymyr_amd: hashset_export_rows: unknown flags");
        if (consumer_stream < -1)
            throw std::invalid_argument("mymyr_amd: hashset_export_rows: invalid consumer stream");
        state_set_sync(set->set);  // the rows [0, size) are complete: no stream handoff is left to do
        int device = 0;
        hip_check(hipPointerGetAttribute(&device, HIP_POINTER_ATTRIBUTE_DEVICE_ORDINAL,
                                         reinterpret_cast<hipDeviceptr_t>(set->set.v.arena)),
                  "hashset_export_rows: device of the arena");
        auto ctx = std::make_unique<Ctx>();
        ctx->shape = {static_cast<int64_t>(set->set.size), static_cast<int64_t>(set->set.v.words)};
        ctx->strides = {static_cast<int64_t>(set->set.v.words), 1};
        set->refs.fetch_add(1, std::memory_order_relaxed);
        ctx->set = set;
        Ctx* c = ctx.release();
        try
        {
            *out = make_managed(set->set.v.arena, device, mya_dl_dtype{MYA_DL_UINT, 64, 1}, c, flags, versioned);
        }
        catch (...)
        {
            c->release();
            delete c;
            throw;
        }
    });
}

void mya_dlpack_capsule_destructor(void* capsule)
{
    using IsValid = int (*)(void*, const char*);
    using GetPointer = void* (*)(void*, const char*);
    static auto* is_valid = reinterpret_cast<IsValid>(dlsym(RTLD_DEFAULT, "PyCapsule_IsValid"));
    static auto* get_pointer = reinterpret_cast<GetPointer>(dlsym(RTLD_DEFAULT, "PyCapsule_GetPointer"));
    if (!capsule || !is_valid || !get_pointer)
        return;
    if (is_valid(capsule, "dltensor_versioned"))
    {
        auto* m = static_cast<mya_dl_managed_versioned*>(get_pointer(capsule, "dltensor_versioned"));
        if (m && m->deleter)
            m->deleter(m);
    }
    else if (is_valid(capsule, "dltensor"))
    {
        auto* m = static_cast<mya_dl_managed*>(get_pointer(capsule, "dltensor"));
        if (m && m->deleter)
            m->deleter(m);
    }
}
}  // extern "C"
