// Host -> device CopyEngines (declared in include/leanstream/hip_copy_engine.h).
#include "leanstream/hip_copy_engine.h"
#include <hip/hip_runtime_api.h>
#include <hsa/hsa.h>
#include <hsa/hsa_ext_amd.h>
#include <cerrno>
#include <stdexcept>
#include <vector>

namespace leanstream::runtime {

// ------------------------------------------------------------------ direct SDMA copies
struct SdmaCopyEngine::Impl {
    hsa_agent_t gpu{}, cpu{};
    std::vector<hsa_signal_t> signals;            // one per lane, 0 = copy complete
    std::vector<hsa_amd_sdma_engine_id_t> ids;    // engines used round robin
    uint64_t chunk = 0;                           // bytes per SDMA copy (0 = one copy per group)
    uint32_t next = 0;
    bool hsa = false;

    struct Find {
        uint32_t domain, bdf;
        hsa_agent_t gpu{}, cpu{};
        bool have_gpu = false, have_cpu = false;
    };
    static hsa_status_t visit(hsa_agent_t agent, void* data) {
        auto& f = *static_cast<Find*>(data);
        hsa_device_type_t type;
        if (hsa_agent_get_info(agent, HSA_AGENT_INFO_DEVICE, &type) != HSA_STATUS_SUCCESS) return HSA_STATUS_SUCCESS;
        if (type == HSA_DEVICE_TYPE_CPU && !f.have_cpu) {
            f.cpu = agent;
            f.have_cpu = true;
        } else if (type == HSA_DEVICE_TYPE_GPU && !f.have_gpu) {
            uint32_t domain = 0, bdf = 0;
            hsa_agent_get_info(agent, static_cast<hsa_agent_info_t>(HSA_AMD_AGENT_INFO_DOMAIN), &domain);
            hsa_agent_get_info(agent, static_cast<hsa_agent_info_t>(HSA_AMD_AGENT_INFO_BDFID), &bdf);
            if (domain == f.domain && (bdf & ~7u) == f.bdf) {   // function bits ignored
                f.gpu = agent;
                f.have_gpu = true;
            }
        }
        return HSA_STATUS_SUCCESS;
    }

    ~Impl() {
        for (hsa_signal_t s : signals) {
            // a copy still in flight keeps writing its signal: wait for it before destroying
            while (hsa_signal_load_scacquire(s) != 0) {
            }
            hsa_signal_destroy(s);
        }
        if (hsa) hsa_shut_down();
    }

    // A group is cut into pieces of `chunk` bytes on successive engines; every piece's
    // completion decrements the lane's signal, which starts at the piece count.
    static int submit(void* c, uint32_t lane, void* dst, const void* src, uint64_t bytes) {
        Impl& m = *static_cast<Impl*>(c);
        if (lane >= m.signals.size()) return EINVAL;
        const uint64_t piece = m.chunk && m.chunk < bytes ? m.chunk : bytes;
        const uint64_t pieces = (bytes + piece - 1) / piece;
        const hsa_signal_t sig = m.signals[lane];
        hsa_signal_store_relaxed(sig, static_cast<hsa_signal_value_t>(pieces));
        for (uint64_t i = 0; i < pieces; ++i) {
            const uint64_t off = i * piece, n = bytes - off < piece ? bytes - off : piece;
            const hsa_amd_sdma_engine_id_t id = m.ids[m.next++ % m.ids.size()];
            const hsa_status_t st =
                hsa_amd_memory_async_copy_on_engine(static_cast<uint8_t*>(dst) + off, m.gpu,
                                                    static_cast<const uint8_t*>(src) + off, m.cpu, n, 0, nullptr, sig,
                                                    id, false);
            if (st != HSA_STATUS_SUCCESS) {
                // retire the pieces never issued, let the issued ones land, then fail
                hsa_signal_subtract_relaxed(sig, static_cast<hsa_signal_value_t>(pieces - i));
                while (hsa_signal_load_scacquire(sig) != 0) {
                }
                return EIO;
            }
        }
        return 0;
    }

    static int poll(void* c, uint32_t lane) {
        Impl& m = *static_cast<Impl*>(c);
        if (lane >= m.signals.size()) return EINVAL;
        return hsa_signal_load_scacquire(m.signals[lane]) == 0 ? 0 : EAGAIN;
    }
};

SdmaCopyEngine::SdmaCopyEngine(int device, uint32_t lanes, uint32_t engines, uint64_t chunk_bytes)
    : impl_(new Impl) {
    Impl& m = *impl_;
    m.chunk = chunk_bytes;
    auto fail = [&](const char* what) {
        delete impl_;
        impl_ = nullptr;
        throw std::runtime_error(what);
    };
    int domain = 0, bus = 0, dev = 0;
    if (!lanes || lanes > 64 || !engines || engines > 16 ||
        hipDeviceGetAttribute(&domain, hipDeviceAttributePciDomainID, device) != hipSuccess ||
        hipDeviceGetAttribute(&bus, hipDeviceAttributePciBusId, device) != hipSuccess ||
        hipDeviceGetAttribute(&dev, hipDeviceAttributePciDeviceId, device) != hipSuccess)
        fail("copy engine geometry");
    if (hsa_init() != HSA_STATUS_SUCCESS) fail("hsa_init");
    m.hsa = true;
    Impl::Find f{static_cast<uint32_t>(domain), static_cast<uint32_t>((bus << 8) | (dev << 3))};
    if (hsa_iterate_agents(Impl::visit, &f) != HSA_STATUS_SUCCESS || !f.have_gpu || !f.have_cpu)
        fail("no HSA agent for the device");
    m.gpu = f.gpu;
    m.cpu = f.cpu;
    uint32_t mask = 0;
    if (hsa_amd_memory_copy_engine_status(m.gpu, m.cpu, &mask) != HSA_STATUS_SUCCESS || !mask)
        fail("no SDMA engine for host to device copies");
    for (uint32_t e = 0; e < 16 && m.ids.size() < engines; ++e)
        if (mask & (1u << e)) m.ids.push_back(static_cast<hsa_amd_sdma_engine_id_t>(1u << e));
    for (uint32_t i = 0; i < lanes; ++i) {
        hsa_signal_t s;
        if (hsa_signal_create(0, 0, nullptr, &s) != HSA_STATUS_SUCCESS) fail("copy signal");
        m.signals.push_back(s);
    }
}

SdmaCopyEngine::~SdmaCopyEngine() { delete impl_; }

CopyEngine SdmaCopyEngine::view() {
    CopyEngine e;
    e.context = impl_;
    e.submit = Impl::submit;
    e.poll = Impl::poll;
    return e;
}

uint32_t SdmaCopyEngine::engines() const { return static_cast<uint32_t>(impl_->ids.size()); }

// ------------------------------------------------------------------ hipMemcpyAsync copies

struct HipCopyEngine::Impl {
    int device = 0;
    std::vector<hipStream_t> streams;
    std::vector<hipEvent_t> events;  // one per lane, recorded after the lane's copy
    uint32_t next = 0;

    ~Impl() {
        for (hipStream_t s : streams) (void)hipStreamSynchronize(s);
        for (hipEvent_t e : events) (void)hipEventDestroy(e);
        for (hipStream_t s : streams) (void)hipStreamDestroy(s);
    }

    // The pump thread issues the copies: bind it to the engine's device once.
    bool on_device() const {
        thread_local int current = -1;
        if (current == device) return true;
        if (hipSetDevice(device) != hipSuccess) return false;
        current = device;
        return true;
    }

    static int submit(void* c, uint32_t lane, void* dst, const void* src, uint64_t bytes) {
        Impl& m = *static_cast<Impl*>(c);
        if (lane >= m.events.size()) return EINVAL;
        if (!m.on_device()) return EIO;
        hipStream_t s = m.streams[m.next++ % m.streams.size()];
        if (hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s) != hipSuccess) return EIO;
        return hipEventRecord(m.events[lane], s) == hipSuccess ? 0 : EIO;
    }

    static int poll(void* c, uint32_t lane) {
        Impl& m = *static_cast<Impl*>(c);
        if (lane >= m.events.size()) return EINVAL;
        const hipError_t q = hipEventQuery(m.events[lane]);
        return q == hipSuccess ? 0 : q == hipErrorNotReady ? EAGAIN : EIO;
    }
};

HipCopyEngine::HipCopyEngine(int device, uint32_t lanes, uint32_t streams) : impl_(new Impl) {
    Impl& m = *impl_;
    m.device = device;
    if (!lanes || lanes > 64 || !streams || streams > kMaxHipCopyStreams || hipSetDevice(device) != hipSuccess) {
        delete impl_;
        throw std::runtime_error("copy engine geometry");
    }
    for (uint32_t i = 0; i < streams; ++i) {
        hipStream_t s = nullptr;
        if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) {
            delete impl_;
            throw std::runtime_error("copy stream");
        }
        m.streams.push_back(s);
    }
    for (uint32_t i = 0; i < lanes; ++i) {
        hipEvent_t e = nullptr;
        if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
            delete impl_;
            throw std::runtime_error("copy event");
        }
        m.events.push_back(e);
    }
}

HipCopyEngine::~HipCopyEngine() { delete impl_; }

CopyEngine HipCopyEngine::view() {
    CopyEngine e;
    e.context = impl_;
    e.submit = Impl::submit;
    e.poll = Impl::poll;
    return e;
}

}  // namespace leanstream::runtime
