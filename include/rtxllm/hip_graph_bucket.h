/* hipGraph replay bucket of the decode runner.
 *
 * Keeps the interface of the reference's CUDA graph bucket
 * (runtime/core/graphs/cuda_graph_bucket.h:14-177): the graph-memory estimate
 * (64 KiB base + 4 KiB per kernel node + 2 KiB per phase + 512 B per
 * batch x query shape, plus a workspace guard of high-water / 64, each aligned),
 * the bucket plan, and an RAII owner of the instantiated graph whose replay()
 * launches it on a stream. Names carry "hip" where the reference's carry
 * "cuda". */
#ifndef RTXLLM_HIP_GRAPH_BUCKET_H
#define RTXLLM_HIP_GRAPH_BUCKET_H

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <limits>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace rtxllm {

struct HipGraphBucketDescriptor {
  std::string name;
  std::uint32_t batch_bucket = 1;
  std::uint32_t query_bucket = 1;
  std::uint32_t phase_count = 0;
  std::uint32_t kernel_launches_per_replay = 0;
  std::size_t workspace_high_water_bytes = 0;
};

struct HipGraphBucketAllocation {
  HipGraphBucketDescriptor descriptor;
  std::size_t offset = 0;
  std::size_t metadata_bytes = 0;
  std::size_t workspace_guard_bytes = 0;
  std::size_t total_bytes = 0;
};

struct HipGraphBucketPlan {
  std::vector<HipGraphBucketAllocation> buckets;
  std::size_t total_bytes = 0;
  std::size_t max_bucket_bytes = 0;
};

namespace graph_bucket_detail {
inline std::size_t add(std::size_t a, std::size_t b) {
  if (a > std::numeric_limits<std::size_t>::max() - b) throw std::overflow_error("hip graph bucket byte count overflow");
  return a + b;
}
inline std::size_t mul(std::size_t a, std::size_t b) {
  if (a != 0 && b > std::numeric_limits<std::size_t>::max() / a)
    throw std::overflow_error("hip graph bucket byte count overflow");
  return a * b;
}
}  // namespace graph_bucket_detail

inline std::size_t align_hip_graph_bucket_bytes(std::size_t value, std::size_t alignment) {
  if (alignment == 0 || (alignment & (alignment - 1)) != 0)
    throw std::invalid_argument("hip graph bucket alignment must be a power of two");
  return graph_bucket_detail::add(value, alignment - 1) & ~(alignment - 1);
}

inline HipGraphBucketAllocation estimate_hip_graph_bucket_allocation(const HipGraphBucketDescriptor& d,
                                                                     std::size_t alignment = 256) {
  using namespace graph_bucket_detail;
  if (d.name.empty()) throw std::invalid_argument("hip graph bucket name must be non-empty");
  if (d.batch_bucket == 0 || d.query_bucket == 0 || d.phase_count == 0 || d.kernel_launches_per_replay == 0)
    throw std::invalid_argument("hip graph bucket dimensions and kernel count must be non-zero");
  std::size_t meta = 64u * 1024u;
  meta = add(meta, mul(d.kernel_launches_per_replay, 4u * 1024u));
  meta = add(meta, mul(d.phase_count, 2u * 1024u));
  meta = add(meta, mul(mul(d.batch_bucket, d.query_bucket), 512u));
  HipGraphBucketAllocation a;
  a.descriptor = d;
  a.metadata_bytes = align_hip_graph_bucket_bytes(meta, alignment);
  a.workspace_guard_bytes = align_hip_graph_bucket_bytes(d.workspace_high_water_bytes / 64u, alignment);
  a.total_bytes = add(a.metadata_bytes, a.workspace_guard_bytes);
  return a;
}

inline HipGraphBucketPlan build_hip_graph_bucket_plan(const std::vector<HipGraphBucketDescriptor>& descriptors,
                                                      std::size_t alignment = 256) {
  if (descriptors.empty()) throw std::invalid_argument("hip graph bucket plan requires at least one bucket");
  HipGraphBucketPlan plan;
  for (const auto& d : descriptors) {
    HipGraphBucketAllocation a = estimate_hip_graph_bucket_allocation(d, alignment);
    a.offset = plan.total_bytes;
    plan.total_bytes = graph_bucket_detail::add(plan.total_bytes, a.total_bytes);
    if (a.total_bytes > plan.max_bucket_bytes) plan.max_bucket_bytes = a.total_bytes;
    plan.buckets.push_back(std::move(a));
  }
  return plan;
}

/* Owns a captured graph and its executable instance. */
class HipGraphBucket {
 public:
  HipGraphBucket() = default;
  HipGraphBucket(const HipGraphBucket&) = delete;
  HipGraphBucket& operator=(const HipGraphBucket&) = delete;
  HipGraphBucket(HipGraphBucket&& o) noexcept : graph_(o.graph_), exec_(o.exec_) { o.graph_ = nullptr, o.exec_ = nullptr; }
  HipGraphBucket& operator=(HipGraphBucket&& o) noexcept {
    if (this != &o) {
      reset();
      graph_ = o.graph_, exec_ = o.exec_;
      o.graph_ = nullptr, o.exec_ = nullptr;
    }
    return *this;
  }
  ~HipGraphBucket() { reset(); }

  /* Takes ownership of `graph` and instantiates it. */
  void instantiate(hipGraph_t graph) {
    reset();
    graph_ = graph;
    const hipError_t st = hipGraphInstantiate(&exec_, graph_, nullptr, nullptr, 0);
    if (st != hipSuccess) {
      exec_ = nullptr;
      throw std::runtime_error(hipGetErrorString(st));
    }
  }
  void replay(hipStream_t stream) const {
    if (!exec_) throw std::logic_error("hip graph bucket has not been instantiated");
    const hipError_t st = hipGraphLaunch(exec_, stream);
    if (st != hipSuccess) throw std::runtime_error(hipGetErrorString(st));
  }
  [[nodiscard]] bool instantiated() const { return exec_ != nullptr; }

 private:
  void reset() noexcept {
    if (exec_) (void)hipGraphExecDestroy(exec_);
    if (graph_) (void)hipGraphDestroy(graph_);
    exec_ = nullptr, graph_ = nullptr;
  }
  hipGraph_t graph_ = nullptr;
  hipGraphExec_t exec_ = nullptr;
};

}  // namespace rtxllm

#endif
