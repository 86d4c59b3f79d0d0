// Step runner: records the kernel launches that a sequence of C-ABI calls
// makes on the calling thread (one decode step), then replays them as
// hand-written AQL kernel-dispatch packets on an HSA queue of its own.
//
// Why: every kernel boundary of a HIP stream or graph carries an agent-scope
// acquire (L1 / scalar-cache invalidation) and an agent-scope release (the
// write-back of every XCD's dirty L2 lines, so that the other XCDs see them).
// The runner writes the same packets, so replaying with those fences matches
// a graph replay; its second fence mode keeps the acquire and drops the
// release for kernels whose outputs are written with agent-scope stores
// (visible to every XCD when the kernel's waves end), which removes the L2
// write-back from every boundary but the last.
//
// The reference replays one captured graph per decode step
// (src/spark_vllm_ascend/plugin/spark2_5.py:369-376 under vLLM's graph
// runner); a replay here is the same unit of work.
#include <hip/hip_runtime.h>
#include <hsa/hsa.h>
#include <hsa/hsa_ext_amd.h>

#include <chrono>
#include <fstream>
#include <iterator>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "../../../include/smx.h"
#include "smx_abi_util.h"
#include "smx_launch.h"

namespace smx {
namespace {
thread_local LaunchSink* t_sink = nullptr;
}
LaunchSink*& launch_sink() { return t_sink; }
}  // namespace smx

namespace {

struct KernelInfo {
  uint64_t object;
  uint32_t kernarg_size, group_size, private_size;
};

struct Packet {
  uint64_t object;
  uint32_t grid[3];  // work-items
  uint16_t block[3];
  uint32_t group_size;
  size_t kernarg_offset;
};

constexpr size_t kKernargAlign = 64;  // each packet's arguments start on a 64-byte boundary

double now_s() {
  return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch())
      .count();
}

struct FindAgent {
  uint32_t bus, device, domain;
  hsa_agent_t gpu{0}, cpu{0};
};

hsa_status_t visit_agent(hsa_agent_t agent, void* data) {
  auto* f = static_cast<FindAgent*>(data);
  hsa_device_type_t type;
  if (hsa_agent_get_info(agent, HSA_AGENT_INFO_DEVICE, &type) != HSA_STATUS_SUCCESS)
    return HSA_STATUS_SUCCESS;
  if (type == HSA_DEVICE_TYPE_CPU && f->cpu.handle == 0) f->cpu = agent;
  if (type != HSA_DEVICE_TYPE_GPU || f->gpu.handle != 0) return HSA_STATUS_SUCCESS;
  uint32_t bdf = 0, domain = 0;
  if (hsa_agent_get_info(agent, (hsa_agent_info_t)HSA_AMD_AGENT_INFO_BDFID, &bdf) !=
          HSA_STATUS_SUCCESS ||
      hsa_agent_get_info(agent, (hsa_agent_info_t)HSA_AMD_AGENT_INFO_DOMAIN, &domain) !=
          HSA_STATUS_SUCCESS)
    return HSA_STATUS_SUCCESS;
  if (((bdf >> 8) & 0xff) == f->bus && ((bdf >> 3) & 0x1f) == f->device && domain == f->domain)
    f->gpu = agent;
  return HSA_STATUS_SUCCESS;
}

struct FindPools {
  hsa_amd_memory_pool_t host{0}, device{0};
};

hsa_status_t visit_cpu_pool(hsa_amd_memory_pool_t pool, void* data) {
  auto* p = static_cast<FindPools*>(data);
  hsa_amd_segment_t seg;
  uint32_t flags = 0;
  if (hsa_amd_memory_pool_get_info(pool, HSA_AMD_MEMORY_POOL_INFO_SEGMENT, &seg) !=
          HSA_STATUS_SUCCESS ||
      seg != HSA_AMD_SEGMENT_GLOBAL)
    return HSA_STATUS_SUCCESS;
  hsa_amd_memory_pool_get_info(pool, HSA_AMD_MEMORY_POOL_INFO_GLOBAL_FLAGS, &flags);
  if ((flags & HSA_AMD_MEMORY_POOL_GLOBAL_FLAG_KERNARG_INIT) && p->host.handle == 0) p->host = pool;
  return HSA_STATUS_SUCCESS;
}

hsa_status_t visit_gpu_pool(hsa_amd_memory_pool_t pool, void* data) {
  auto* p = static_cast<FindPools*>(data);
  hsa_amd_segment_t seg;
  uint32_t flags = 0;
  if (hsa_amd_memory_pool_get_info(pool, HSA_AMD_MEMORY_POOL_INFO_SEGMENT, &seg) !=
          HSA_STATUS_SUCCESS ||
      seg != HSA_AMD_SEGMENT_GLOBAL)
    return HSA_STATUS_SUCCESS;
  hsa_amd_memory_pool_get_info(pool, HSA_AMD_MEMORY_POOL_INFO_GLOBAL_FLAGS, &flags);
  if ((flags & HSA_AMD_MEMORY_POOL_GLOBAL_FLAG_COARSE_GRAINED) && p->device.handle == 0)
    p->device = pool;
  return HSA_STATUS_SUCCESS;
}

struct SymbolScan {
  hsa_executable_t exe;
  std::unordered_map<std::string, KernelInfo>* out;
  std::unordered_set<std::string>* ambiguous;  // names found in more than one code object
};

hsa_status_t visit_symbol(hsa_executable_t, hsa_agent_t, hsa_executable_symbol_t sym, void* data) {
  auto* s = static_cast<SymbolScan*>(data);
  hsa_symbol_kind_t kind;
  if (hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_TYPE, &kind) !=
          HSA_STATUS_SUCCESS ||
      kind != HSA_SYMBOL_KIND_KERNEL)
    return HSA_STATUS_SUCCESS;
  uint32_t len = 0;
  hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_NAME_LENGTH, &len);
  std::string name(len, '\0');
  hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_NAME, name.data());
  if (name.size() > 3 && name.compare(name.size() - 3, 3, ".kd") == 0)
    name.resize(name.size() - 3);
  KernelInfo k{};
  hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_OBJECT, &k.object);
  hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_KERNARG_SEGMENT_SIZE,
                                 &k.kernarg_size);
  hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_GROUP_SEGMENT_SIZE,
                                 &k.group_size);
  hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_PRIVATE_SEGMENT_SIZE,
                                 &k.private_size);
  if (!s->out->emplace(name, k).second) s->ambiguous->insert(name);
  return HSA_STATUS_SUCCESS;
}

void queue_error(hsa_status_t status, hsa_queue_t*, void*) {
  // The queue is unusable after an error; report it (the process's HSA
  // runtime aborts on its own for errors it treats as fatal).
  const char* msg = "unknown";
  hsa_status_string(status, &msg);
  fprintf(stderr, "smx step runner: HSA queue error: %s\n", msg);
}

}  // namespace

struct smx_runner final : smx::LaunchSink {
  hsa_agent_t gpu{0};
  FindPools pools;
  // the code objects' bytes stay alive with the runner: the loader (and the
  // tools that inspect loaded code objects) may refer to the memory they
  // were loaded from
  std::vector<std::vector<char>> blobs;
  std::vector<hsa_code_object_reader_t> readers;
  std::vector<hsa_executable_t> executables;
  std::unordered_map<std::string, KernelInfo> kernels;
  std::unordered_set<std::string> ambiguous;
  hsa_queue_t* queue = nullptr;
  hsa_signal_t pending{0};  // decremented by the last packet of each replay
  hsa_signal_t first{0};    // completion signal of the first packet (timing)
  uint64_t last_total = 0;  // packets of the last replay
  bool hsa_up = false;
  // set when a replay could not write all its packets (the queue did not
  // drain): its last packet, which would bring `pending` back to 0, was never
  // written, so the runner refuses every later call and is never freed (the
  // packets already written may still read its kernel arguments)
  std::string broken;
  double drain_timeout_s = 30.0;  // how long a replay waits for a free queue slot

  // recording
  bool recording = false;
  std::string record_error;
  std::vector<Packet> packets;
  std::vector<unsigned char> kernarg_host;
  // replay
  void* kernarg_dev = nullptr;
  size_t kernarg_dev_size = 0;
  bool ready = false;

  void record(const void* host_fn, dim3 grid, dim3 block, uint32_t dynamic_lds,
              const void* kernarg, size_t kernarg_size) override {
    if (!record_error.empty()) return;
    const char* name = hipKernelNameRefByPtr(host_fn, nullptr);
    if (!name) {
      record_error = "a recorded launch names no known kernel";
      return;
    }
    auto it = kernels.find(name);
    if (it == kernels.end()) {
      record_error = std::string("kernel not in the runner's code objects: ") + name;
      return;
    }
    if (ambiguous.count(name)) {
      record_error = std::string("kernel defined in more than one code object: ") + name;
      return;
    }
    const KernelInfo& k = it->second;
    // explicit arguments only: a larger segment means implicit arguments,
    // which the runner does not fill
    if (kernarg_size > smx::kMaxKernarg || k.kernarg_size < kernarg_size ||
        k.kernarg_size > ((kernarg_size + 15) & ~size_t(15))) {
      record_error = std::string("kernel argument layout not supported: ") + name;
      return;
    }
    if (k.private_size != 0) {
      record_error = std::string("kernel needs scratch memory: ") + name;
      return;
    }
    const uint64_t gx = (uint64_t)grid.x * block.x, gy = (uint64_t)grid.y * block.y,
                   gz = (uint64_t)grid.z * block.z;
    if (gx == 0 || gy == 0 || gz == 0 || gx > UINT32_MAX || gy > UINT32_MAX || gz > UINT32_MAX ||
        (uint64_t)block.x * block.y * block.z > 1024) {
      record_error = std::string("launch shape out of range: ") + name;
      return;
    }
    Packet p{};
    p.object = k.object;
    p.grid[0] = (uint32_t)gx;
    p.grid[1] = (uint32_t)gy;
    p.grid[2] = (uint32_t)gz;
    p.block[0] = (uint16_t)block.x;
    p.block[1] = (uint16_t)block.y;
    p.block[2] = (uint16_t)block.z;
    p.group_size = k.group_size + dynamic_lds;
    p.kernarg_offset = kernarg_host.size();
    kernarg_host.resize(kernarg_host.size() +
                            ((k.kernarg_size + kKernargAlign - 1) & ~(kKernargAlign - 1)),
                        0);
    memcpy(kernarg_host.data() + p.kernarg_offset, kernarg, kernarg_size);
    packets.push_back(p);
  }

  void release_kernargs() {
    if (kernarg_dev) hsa_amd_memory_pool_free(kernarg_dev);
    kernarg_dev = nullptr;
    kernarg_dev_size = 0;
    ready = false;
  }

  ~smx_runner() {
    release_kernargs();
    if (pending.handle) hsa_signal_destroy(pending);
    if (first.handle) hsa_signal_destroy(first);
    if (queue) hsa_queue_destroy(queue);
    for (auto e : executables) hsa_executable_destroy(e);
    for (auto r : readers) hsa_code_object_reader_destroy(r);
    if (hsa_up) hsa_shut_down();
  }
};

namespace {

int fail(const char* func, const std::string& msg) {
  smx::set_last_error(func, msg.c_str());
  return SMX_EINVAL;
}

#define HSA_OR_FAIL(call, what)                                              \
  do {                                                                       \
    if ((call) != HSA_STATUS_SUCCESS) return fail(__func__, (what));         \
  } while (0)

}  // namespace

extern "C" int smx_runner_create(const char* const* code_objects, int32_t count,
                                 smx_runner** out) {
  SMX_REQUIRE(out && code_objects && count >= 1 && count <= 64, "need 1..64 code objects");
  *out = nullptr;
  int dev = 0, bus = 0, device = 0, domain = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&bus, hipDeviceAttributePciBusId, dev) != hipSuccess ||
      hipDeviceGetAttribute(&device, hipDeviceAttributePciDeviceId, dev) != hipSuccess ||
      hipDeviceGetAttribute(&domain, hipDeviceAttributePciDomainId, dev) != hipSuccess)
    return fail(__func__, "no current HIP device");
  auto* r = new smx_runner();
  auto bail = [&](const std::string& msg) {
    delete r;
    return fail("smx_runner_create", msg);
  };
  if (hsa_init() != HSA_STATUS_SUCCESS) return bail("hsa_init failed");
  r->hsa_up = true;
  FindAgent fa{(uint32_t)bus, (uint32_t)device, (uint32_t)domain};
  if (hsa_iterate_agents(visit_agent, &fa) != HSA_STATUS_SUCCESS || !fa.gpu.handle ||
      !fa.cpu.handle)
    return bail("no HSA agent for the current HIP device");
  r->gpu = fa.gpu;
  if (hsa_amd_agent_iterate_memory_pools(fa.cpu, visit_cpu_pool, &r->pools) != HSA_STATUS_SUCCESS ||
      hsa_amd_agent_iterate_memory_pools(fa.gpu, visit_gpu_pool, &r->pools) != HSA_STATUS_SUCCESS ||
      !r->pools.host.handle || !r->pools.device.handle)
    return bail("no kernarg or device memory pool");
  for (int i = 0; i < count; ++i) {
    if (!code_objects[i]) return bail("null code object path");
    std::ifstream f(code_objects[i], std::ios::binary);
    r->blobs.emplace_back((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    const std::vector<char>& blob = r->blobs.back();
    if (blob.empty()) return bail(std::string("cannot read ") + code_objects[i]);
    hsa_code_object_reader_t reader;
    if (hsa_code_object_reader_create_from_memory(blob.data(), blob.size(), &reader) !=
        HSA_STATUS_SUCCESS)
      return bail(std::string("not a code object: ") + code_objects[i]);
    r->readers.push_back(reader);
    hsa_executable_t exe;
    if (hsa_executable_create_alt(HSA_PROFILE_FULL, HSA_DEFAULT_FLOAT_ROUNDING_MODE_DEFAULT,
                                  nullptr, &exe) != HSA_STATUS_SUCCESS)
      return bail("hsa_executable_create_alt failed");
    r->executables.push_back(exe);
    if (hsa_executable_load_agent_code_object(exe, r->gpu, reader, nullptr, nullptr) !=
            HSA_STATUS_SUCCESS ||
        hsa_executable_freeze(exe, nullptr) != HSA_STATUS_SUCCESS)
      return bail(std::string("cannot load ") + code_objects[i]);
    SymbolScan scan{exe, &r->kernels, &r->ambiguous};
    if (hsa_executable_iterate_agent_symbols(exe, r->gpu, visit_symbol, &scan) !=
        HSA_STATUS_SUCCESS)
      return bail("cannot list kernels");
  }
  uint32_t qmax = 0;
  hsa_agent_get_info(r->gpu, HSA_AGENT_INFO_QUEUE_MAX_SIZE, &qmax);
  const uint32_t qsize = qmax >= 16384 ? 16384 : qmax;
  if (qsize < 256) return bail("HSA queue too small");
  if (hsa_queue_create(r->gpu, qsize, HSA_QUEUE_TYPE_SINGLE, queue_error, nullptr, UINT32_MAX,
                       UINT32_MAX, &r->queue) != HSA_STATUS_SUCCESS)
    return bail("hsa_queue_create failed");
  if (hsa_signal_create(0, 0, nullptr, &r->pending) != HSA_STATUS_SUCCESS ||
      hsa_signal_create(0, 0, nullptr, &r->first) != HSA_STATUS_SUCCESS)
    return bail("hsa_signal_create failed");
  // packet-processor timestamps on the packets that carry a completion
  // signal (the first and the last of a replay): smx_runner_elapsed
  if (hsa_amd_profiling_set_profiler_enabled(r->queue, 1) != HSA_STATUS_SUCCESS)
    return bail("cannot enable queue timestamps");
  *out = r;
  return 0;
}

#define SMX_REQUIRE_WORKING(r)                                                   \
  do {                                                                           \
    if (!(r)->broken.empty()) return fail(__func__, "the runner is broken: " + (r)->broken); \
  } while (0)

extern "C" int smx_runner_begin(smx_runner* r) {
  SMX_REQUIRE(r, "null runner");
  SMX_REQUIRE_WORKING(r);
  SMX_REQUIRE(!smx::launch_sink(), "this thread is already recording");
  SMX_REQUIRE(hsa_signal_load_scacquire(r->pending) == 0, "a replay is still running");
  r->release_kernargs();
  r->packets.clear();
  r->kernarg_host.clear();
  r->record_error.clear();
  r->recording = true;
  smx::launch_sink() = r;
  return 0;
}

extern "C" int smx_runner_end(smx_runner* r) {
  SMX_REQUIRE(r && r->recording, "the runner is not recording");
  SMX_REQUIRE(smx::launch_sink() == r, "recording was started on another thread");
  smx::launch_sink() = nullptr;
  r->recording = false;
  if (!r->record_error.empty()) return fail(__func__, r->record_error);
  if (r->packets.empty()) return fail(__func__, "nothing was recorded");
  const size_t bytes = r->kernarg_host.size();
  void* staging = nullptr;
  HSA_OR_FAIL(hsa_amd_memory_pool_allocate(r->pools.device, bytes, 0, &r->kernarg_dev),
              "cannot allocate kernel arguments");
  r->kernarg_dev_size = bytes;
  HSA_OR_FAIL(hsa_amd_memory_pool_allocate(r->pools.host, bytes, 0, &staging),
              "cannot allocate staging memory");
  memcpy(staging, r->kernarg_host.data(), bytes);
  const bool ok = hsa_amd_agents_allow_access(1, &r->gpu, nullptr, staging) ==
                      HSA_STATUS_SUCCESS &&
                  hsa_memory_copy(r->kernarg_dev, staging, bytes) == HSA_STATUS_SUCCESS;
  hsa_amd_memory_pool_free(staging);
  if (!ok) return fail(__func__, "cannot upload kernel arguments");
  r->ready = true;
  return 0;
}

extern "C" int smx_runner_num_packets(const smx_runner* r, int64_t* out) {
  SMX_REQUIRE(r && out, "null argument");
  *out = (int64_t)r->packets.size();
  return 0;
}

extern "C" int smx_runner_replay(smx_runner* r, int32_t repeats, int32_t fences) {
  SMX_REQUIRE(r, "null runner");
  SMX_REQUIRE_WORKING(r);
  SMX_REQUIRE(r->ready, "nothing recorded");
  SMX_REQUIRE(repeats >= 1 && repeats <= 1000000, "repeats must be in [1, 1e6]");
  SMX_REQUIRE(fences == SMX_RUNNER_FENCES_AGENT || fences == SMX_RUNNER_FENCES_ACQUIRE_ONLY,
              "unknown fence mode");
  hsa_queue_t* q = r->queue;
  const uint32_t mask = q->size - 1;
  const uint64_t total = (uint64_t)repeats * r->packets.size();
  auto* base = static_cast<hsa_kernel_dispatch_packet_t*>(q->base_address);
  const int acq = HSA_FENCE_SCOPE_AGENT;
  const int rel = fences == SMX_RUNNER_FENCES_AGENT ? HSA_FENCE_SCOPE_AGENT : HSA_FENCE_SCOPE_NONE;
  hsa_signal_add_screlease(r->pending, 1);
  if (total > 1) hsa_signal_store_relaxed(r->first, 1);
  r->last_total = total;
  uint64_t idx = 0;
  for (uint64_t i = 0; i < total; ++i) {
    // wait (bounded) for a free slot before claiming it: the packet processor
    // frees a slot when it has consumed the packet written q->size packets
    // earlier.  The queue has one producer (this runner, one call at a time),
    // so the index seen here is the one the claim below returns.
    const uint64_t next = hsa_queue_load_write_index_relaxed(q);
    if (next - hsa_queue_load_read_index_scacquire(q) >= q->size) {
      if (i > 0)  // let the packet processor see this replay's packets so far
        hsa_signal_store_screlease(q->doorbell_signal, (hsa_signal_value_t)(next - 1));
      const double t0 = now_s();
      while (next - hsa_queue_load_read_index_scacquire(q) >= q->size) {
        if (now_s() - t0 > r->drain_timeout_s) {
          // nothing claimed; the packets already written still run, but the
          // replay's last packet (the one that signals `pending`) is never
          // written, so the runner cannot be waited on or reused
          r->broken = "a replay stopped after " + std::to_string(i) + " of " +
                      std::to_string(total) + " packets: the queue did not drain in time";
          return fail(__func__, r->broken);
        }
      }
    }
    idx = hsa_queue_add_write_index_relaxed(q, 1);
    const Packet& p = r->packets[i % r->packets.size()];
    hsa_kernel_dispatch_packet_t* d = base + (idx & mask);
    d->workgroup_size_x = p.block[0];
    d->workgroup_size_y = p.block[1];
    d->workgroup_size_z = p.block[2];
    d->reserved0 = 0;
    d->grid_size_x = p.grid[0];
    d->grid_size_y = p.grid[1];
    d->grid_size_z = p.grid[2];
    d->private_segment_size = 0;
    d->group_segment_size = p.group_size;
    d->kernel_object = p.object;
    d->kernarg_address = static_cast<char*>(r->kernarg_dev) + p.kernarg_offset;
    d->reserved2 = 0;
    const bool first = i == 0, last = i + 1 == total;
    d->completion_signal = last ? r->pending : first ? r->first : hsa_signal_t{0};
    // the first packet sees everything the host and HIP streams completed;
    // the last one makes every result visible to the host
    const int a = first ? HSA_FENCE_SCOPE_SYSTEM : acq;
    const int l = last ? HSA_FENCE_SCOPE_SYSTEM : rel;
    const uint16_t header = (uint16_t)((HSA_PACKET_TYPE_KERNEL_DISPATCH << HSA_PACKET_HEADER_TYPE) |
                                       (1 << HSA_PACKET_HEADER_BARRIER) |
                                       (a << HSA_PACKET_HEADER_SCACQUIRE_FENCE_SCOPE) |
                                       (l << HSA_PACKET_HEADER_SCRELEASE_FENCE_SCOPE));
    const uint16_t setup = (uint16_t)(3 << HSA_KERNEL_DISPATCH_PACKET_SETUP_DIMENSIONS);
    __atomic_store_n(reinterpret_cast<uint32_t*>(d), (uint32_t)header | ((uint32_t)setup << 16),
                     __ATOMIC_RELEASE);
    if ((i & 255) == 255) hsa_signal_store_screlease(q->doorbell_signal, (hsa_signal_value_t)idx);
  }
  hsa_signal_store_screlease(q->doorbell_signal, (hsa_signal_value_t)idx);
  return 0;
}

extern "C" int smx_runner_set_drain_timeout(smx_runner* r, double seconds) {
  SMX_REQUIRE(r, "null runner");
  SMX_REQUIRE(seconds >= 0.0 && seconds <= 3600.0, "seconds must be in [0, 3600]");
  r->drain_timeout_s = seconds;
  return 0;
}

extern "C" int smx_runner_wait(smx_runner* r, double timeout_s) {
  SMX_REQUIRE(r, "null runner");
  SMX_REQUIRE_WORKING(r);
  SMX_REQUIRE(timeout_s > 0.0, "timeout must be positive");
  const double t0 = now_s();
  while (hsa_signal_wait_scacquire(r->pending, HSA_SIGNAL_CONDITION_EQ, 0, 1000000,
                                   HSA_WAIT_STATE_ACTIVE) != 0) {
    if (now_s() - t0 > timeout_s) return fail(__func__, "replay did not complete in time");
  }
  return 0;
}

extern "C" int smx_runner_elapsed(smx_runner* r, double* seconds) {
  SMX_REQUIRE(r && seconds, "null argument");
  SMX_REQUIRE_WORKING(r);
  SMX_REQUIRE(r->last_total > 0, "nothing replayed");
  SMX_REQUIRE(hsa_signal_load_scacquire(r->pending) == 0, "a replay is still running");
  hsa_amd_profiling_dispatch_time_t t_first{}, t_last{};
  HSA_OR_FAIL(hsa_amd_profiling_get_dispatch_time(r->gpu, r->pending, &t_last),
              "no timestamps for the last packet");
  if (r->last_total > 1) {
    HSA_OR_FAIL(hsa_amd_profiling_get_dispatch_time(r->gpu, r->first, &t_first),
                "no timestamps for the first packet");
  } else {
    t_first = t_last;
  }
  uint64_t freq = 0;
  HSA_OR_FAIL(hsa_system_get_info(HSA_SYSTEM_INFO_TIMESTAMP_FREQUENCY, &freq),
              "no timestamp frequency");
  SMX_REQUIRE(freq > 0 && t_last.end >= t_first.start, "inconsistent timestamps");
  *seconds = (double)(t_last.end - t_first.start) / (double)freq;
  return 0;
}

extern "C" void smx_runner_destroy(smx_runner* r) {
  if (!r) return;
  if (smx::launch_sink() == r) smx::launch_sink() = nullptr;
  // never free memory a running replay reads: wait for it (bounded) first,
  // and leak the runner if it does not drain -- or if a replay broke it, as
  // its `pending` count never returns to 0
  if (!r->broken.empty()) {
    fprintf(stderr, "smx step runner: %s; the runner is not freed\n", r->broken.c_str());
    return;
  }
  if (hsa_signal_load_scacquire(r->pending) != 0 && smx_runner_wait(r, 60.0) != 0) {
    fprintf(stderr, "smx step runner: a replay still runs after 60 s; the runner is not freed\n");
    return;
  }
  delete r;
}

extern "C" int smx_graph_num_nodes(void* graph, int64_t* count) {
  SMX_REQUIRE(graph && count, "null argument");
  size_t n = 0;
  const hipError_t e = hipGraphGetNodes(static_cast<hipGraph_t>(graph), nullptr, &n);
  if (e != hipSuccess) return (int)e;
  *count = (int64_t)n;
  return 0;
}
