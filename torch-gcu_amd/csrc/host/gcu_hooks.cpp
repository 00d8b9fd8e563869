// PrivateUse1 hooks, the device generator and static registration of the
// allocator (the reference's GCUHooks, torch_gcu/csrc/gcu/gcu_hooks.cpp:17-139,
// and static init, gcu_custom_api.cpp:35-42 / gcu_context.cpp:60-62).
#include <ATen/EmptyTensor.h>
#include <ATen/core/GeneratorForPrivateuseone.h>
#include <ATen/detail/PrivateUse1HooksInterface.h>
#include <c10/core/CPUAllocator.h>
#include <c10/core/GeneratorImpl.h>
#include <c10/core/impl/alloc_cpu.h>

#include <atomic>
#include <mutex>
#include <vector>

#include "gcu_caching_allocator.h"
#include "gcu_caching_host_allocator.h"
#include "gcu_runtime.h"
#include "mi355x_ops.h"

namespace torch_gcu {

// Philox seed/offset bookkeeping of a gcu device.  Random-number ops run on
// the CPU (there is no device RNG kernel on this path), so the generator only
// keeps state: manual_seed / initial_seed / get_state / set_state work and a
// graph can record the offset (torch_gcu/csrc/gcu/gcu_generator_impl.h:27-80).
struct GCUGeneratorImpl : public c10::GeneratorImpl {
  explicit GCUGeneratorImpl(c10::DeviceIndex d)
      : c10::GeneratorImpl(c10::Device(kGCU, d), c10::DispatchKeySet(c10::DispatchKey::PrivateUse1)) {}
  void set_current_seed(uint64_t seed) override {
    seed_ = seed;
    offset_ = 0;
  }
  void set_offset(uint64_t offset) override { offset_ = offset; }
  uint64_t get_offset() const override { return offset_; }
  uint64_t current_seed() const override { return seed_; }
  uint64_t seed() override {
    const uint64_t s = c10::detail::getNonDeterministicRandom(true);
    set_current_seed(s);
    return s;
  }
  void set_state(const c10::TensorImpl& state) override {
    TORCH_CHECK(state.numel() == 16 && state.dtype() == caffe2::TypeMeta::Make<uint8_t>(),
                "gcu generator state must be a 16-byte uint8 tensor");
    const uint8_t* p = static_cast<const uint8_t*>(state.data());
    std::memcpy(&seed_, p, 8);
    std::memcpy(&offset_, p + 8, 8);
  }
  c10::intrusive_ptr<c10::TensorImpl> get_state() const override {
    auto t = at::detail::empty_cpu({16}, at::kByte, std::nullopt, std::nullopt, std::nullopt,
                                   std::nullopt);
    uint8_t* p = t.data_ptr<uint8_t>();
    std::memcpy(p, &seed_, 8);
    std::memcpy(p + 8, &offset_, 8);
    return t.getIntrusivePtr();
  }
  // Reserves `increment` Philox counters and returns the previous offset.
  uint64_t philox_advance(uint64_t increment) {
    const uint64_t o = offset_;
    offset_ += (increment + 3) / 4 * 4;
    return o;
  }
  static c10::DeviceType device_type() { return kGCU; }

 private:
  GCUGeneratorImpl* clone_impl() const override {
    auto* g = new GCUGeneratorImpl(device().index());
    g->seed_ = seed_;
    g->offset_ = offset_;
    return g;
  }
  uint64_t seed_ = 67280421310721ULL;
  uint64_t offset_ = 0;
};

// The caching allocator as the kernel library's stream-ordered workspace
// allocator (gcu_custom_api.cpp:23-31 registers the reference's the same way).
void register_library_workspace() {
  mi_set_workspace_allocator(reinterpret_cast<mi_alloc_fn>(&allocator::workspace_alloc),
                             reinterpret_cast<mi_free_fn>(&allocator::workspace_free), nullptr);
}

namespace {

std::mutex g_gen_mu;
std::atomic<bool> g_initialized{false};
std::vector<at::Generator> g_default_gens;

struct GCUHooks final : public at::PrivateUse1HooksInterface {
  bool isBuilt() const override { return true; }
  bool isAvailable() const override { return device_count() > 0; }
  bool hasPrimaryContext(c10::DeviceIndex) const override { return true; }

  void init() const override {
    static std::once_flag once;
    std::call_once(once, [] {
      g_initialized.store(true);
      allocator::init(device_count());
      register_library_workspace();
    });
  }

  const at::Generator& getDefaultGenerator(c10::DeviceIndex d) const override {
    std::lock_guard<std::mutex> g(g_gen_mu);
    const int n = std::max<int>(1, device_count());
    if (g_default_gens.empty()) {
      for (int i = 0; i < n; ++i)
        g_default_gens.push_back(at::make_generator<GCUGeneratorImpl>((c10::DeviceIndex)i));
    }
    if (d < 0) d = current_device();
    TORCH_CHECK(d < (int)g_default_gens.size(), "gcu: invalid device index ", (int)d);
    return g_default_gens[d];
  }

  at::Generator getNewGenerator(c10::DeviceIndex d) const override {
    return at::make_generator<GCUGeneratorImpl>(d < 0 ? current_device() : d);
  }

  at::Device getDeviceFromPtr(void* data) const override {
    hipPointerAttribute_t attr;
    GCU_HIP_CHECK(hipPointerGetAttributes(&attr, data));
    return at::Device(kGCU, (c10::DeviceIndex)attr.device);
  }

  // Blocks of the caching host allocator, and any other page-locked memory
  // HIP knows of (gcu_hooks.cpp:39-58 asks the runtime the same way).
  bool isPinnedPtr(const void* data) const override {
    if (data == nullptr) return false;
    if (host_allocator::owns(data)) return true;
    if (allocator::host_memory_mode() || device_count() == 0) return false;
    hipPointerAttribute_t attr;
    const hipError_t e = hipPointerGetAttributes(&attr, data);
    if (e != hipSuccess) {
      (void)hipGetLastError();  // pageable memory is not known to HIP
      return false;
    }
    return attr.type == hipMemoryTypeHost;
  }

  at::Allocator* getPinnedMemoryAllocator() const override { return host_allocator::get(); }

  void resizePrivateUse1Bytes(const c10::Storage& storage, size_t newsize) const override {
    c10::StorageImpl* impl = storage.unsafeGetStorageImpl();
    TORCH_CHECK(impl->resizable(), "Trying to resize storage that is not resizable");
    at::DataPtr fresh = allocator::get()->allocate(newsize);
    const size_t keep = std::min(newsize, storage.nbytes());
    if (keep > 0 && storage.data() != nullptr)
      GCU_HIP_CHECK(hipMemcpyAsync(fresh.get(), storage.data(), keep, hipMemcpyDeviceToDevice,
                                   current_hip_stream()));
    impl->set_data_ptr_noswap(std::move(fresh));
    impl->set_nbytes(newsize);
  }
};

GCUHooks* g_hooks = nullptr;

const bool g_registered = [] {
  g_hooks = new GCUHooks();
  at::RegisterPrivateUse1HooksInterface(g_hooks);
  c10::SetAllocator(kGCU, allocator::get());
  return true;
}();

}  // namespace

void ensure_initialized() { g_hooks->init(); }

bool is_initialized() { return g_initialized.load(); }

}  // namespace torch_gcu
