// Neighbourhoods within a geodesic radius and their per-edge geometry, built on
// the GPU from float64 node coordinates.
//
// Membership is the reference's exact rule (discretization/edge_geometry.py:
// 381-387, 492-503): target i and source j are neighbours iff
//   atan2(|p_i x q_j|, clamp(<p_i, q_j>, -1, 1)) <= limit   (limit = r + 1e-10)
// evaluated in float64 with every product rounded on its own and the sums
// taken left to right.  Candidates come from 64-node bounding boxes instead of
// a KD-tree: a wavefront owns 64 consecutive targets and walks the source boxes
// in increasing index, skipping a box only when it lies farther than the chord
// of the limit on some axis (a Euclidean bound, so no neighbour is skipped).
// For unit vectors the computed <p, q> lies within about 1e-15 of cos(angle),
// and the computed geodesic within a few 1e-15 of the angle, so a dot product
// more than 1e-12 above cos(limit) is inside and one more than 1e-12 below is
// outside, whatever atan2 would round to: only pairs in that band take the
// exact test, and the decisions are the exact test's.  Each lane appends its target's neighbours in increasing source
// index, so rows come out target-major, source-minor (:701-704) without a sort.
// Two passes: degrees (then an in-place prefix sum into row_ptr, :622-653),
// then the edge list into the rows the caller sized from row_ptr[n].
//
// The per-edge tables (edge_geometry_from_index, :506-619) are one pass per
// edge: log map in the target frame, geodesic distance, Levi-Civita transport
// angle, tangent quadrature weight, polar angle, and both phase tables.
#include <algorithm>

#include "common.hpp"

namespace gm {
namespace {

constexpr int kGeoTile = 64;         // nodes per bounding box = targets per wavefront
constexpr int kScanThreads = 1024;   // one workgroup turns the degrees into row_ptr
constexpr int kTableThreads = 256;

__device__ __forceinline__ int64_t imin(int64_t x, int64_t y) { return x < y ? x : y; }

// In-wave LDS hand-off: stores before, loads after, with no reordering across it.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ double wave_min(double v) {
  for (int o = 32; o; o >>= 1) v = fmin(v, __shfl_xor(v, o, kWave));
  return v;
}
__device__ __forceinline__ double wave_max(double v) {
  for (int o = 32; o; o >>= 1) v = fmax(v, __shfl_xor(v, o, kWave));
  return v;
}

// <p, q> with each product rounded and the sum taken left to right.
__device__ __forceinline__ double dot3(const double* p, const double* q) {
#pragma clang fp contract(off)
  return p[0] * q[0] + p[1] * q[1] + p[2] * q[2];
}

// p x q, each product rounded.
__device__ __forceinline__ void cross3(const double* p, const double* q, double* c) {
#pragma clang fp contract(off)
  c[0] = p[1] * q[2] - p[2] * q[1];
  c[1] = p[2] * q[0] - p[0] * q[2];
  c[2] = p[0] * q[1] - p[1] * q[0];
}

__device__ __forceinline__ double norm3(const double* c) {
#pragma clang fp contract(off)
  return sqrt(c[0] * c[0] + c[1] * c[1] + c[2] * c[2]);
}

__device__ __forceinline__ double clamp_unit(double x) { return fmin(fmax(x, -1.0), 1.0); }

// atan2(|p x q|, clamp(<p, q>)), given the unclamped <p, q>.
__device__ __forceinline__ double geodesic(const double* p, const double* q, double dot) {
  double c[3];
  cross3(p, q, c);
  return atan2(norm3(c), clamp_unit(dot));
}

__global__ __launch_bounds__(kGeoTile) void geo_bounds_kernel(const double* __restrict__ nodes, int64_t n,
                                                              double* __restrict__ boxes) {
  const int64_t tile = blockIdx.x;
  const int lane = threadIdx.x;
  const int64_t i = imin(tile * kGeoTile + lane, n - 1);  // lanes past the end repeat the last node
  double lo[3], hi[3];
  for (int k = 0; k < 3; ++k) {
    const double x = nodes[3 * i + k];
    lo[k] = wave_min(x);
    hi[k] = wave_max(x);
  }
  if (lane == 0) {
    for (int k = 0; k < 3; ++k) {
      boxes[6 * tile + k] = lo[k];
      boxes[6 * tile + 3 + k] = hi[k];
    }
  }
}

struct WalkArgs {
  const double* targets;
  const double* sources;
  const double* target_boxes;
  const double* source_boxes;
  int64_t n_targets, n_sources;
  double limit;      // membership: geodesic <= limit
  double cos_floor;  // pairs with <p, q> below this are farther than the limit
  double cos_in;     // pairs with <p, q> at or above this are within the limit
  double reach;      // chord of the limit plus a margin: the box test's distance
  int64_t* row_ptr;  // degree pass: degree of t at row_ptr[t + 1]; edge pass: row offsets (read only)
  int64_t* target_out;
  int64_t* source_out;
  int64_t n_edges;   // edge pass: capacity of target_out / source_out
};

template <bool kEdges>
__global__ __launch_bounds__(kGeoTile) void geo_walk_kernel(WalkArgs a) {
  __shared__ double pts[kGeoTile][4];
  const int lane = threadIdx.x;
  const int64_t tile = xcd_block(blockIdx.x, gridDim.x);
  const int64_t t = tile * kGeoTile + lane;
  const bool valid = t < a.n_targets;
  const int64_t tt = valid ? t : a.n_targets - 1;
  const double p[3] = {a.targets[3 * tt], a.targets[3 * tt + 1], a.targets[3 * tt + 2]};
  double tlo[3], thi[3];
  for (int k = 0; k < 3; ++k) {
    tlo[k] = a.target_boxes[6 * tile + k];
    thi[k] = a.target_boxes[6 * tile + 3 + k];
  }
  int64_t pos = 0, end = 0, count = 0;
  if (kEdges && valid) {
    pos = a.row_ptr[t];
    end = imin(a.row_ptr[t + 1], a.n_edges);
  }
  const int64_t source_tiles = (a.n_sources + kGeoTile - 1) / kGeoTile;
  for (int64_t st = 0; st < source_tiles; ++st) {
    const double* box = a.source_boxes + 6 * st;
    bool apart = false;
    for (int k = 0; k < 3; ++k) apart |= (box[k] - a.reach > thi[k]) || (tlo[k] - a.reach > box[3 + k]);
    if (apart) continue;
    const int64_t j0 = st * kGeoTile;
    const int m = (int)imin(kGeoTile, a.n_sources - j0);
    wave_sync();  // the previous tile's reads are done before it is overwritten
    if (lane < m) {
      for (int k = 0; k < 3; ++k) pts[lane][k] = a.sources[3 * (j0 + lane) + k];
    }
    wave_sync();
    for (int s = 0; s < m; ++s) {
      const double q[3] = {pts[s][0], pts[s][1], pts[s][2]};
      const double dot = dot3(p, q);
      if (valid && dot >= a.cos_floor) {
        if (dot >= a.cos_in || geodesic(p, q, dot) <= a.limit) {
          if (kEdges) {
            if (pos < end) {
              a.target_out[pos] = t;
              a.source_out[pos] = j0 + s;
            }
            ++pos;
          } else {
            ++count;
          }
        }
      }
    }
  }
  if (!kEdges && valid) a.row_ptr[t + 1] = count;
}

// row_ptr[1..n] holds the degrees; leaves their inclusive prefix sums there and 0 in row_ptr[0].
__global__ __launch_bounds__(kScanThreads) void geo_scan_kernel(int64_t* __restrict__ row_ptr, int64_t n) {
  __shared__ int64_t sums[kScanThreads];
  const int tid = threadIdx.x;
  const int64_t chunk = (n + kScanThreads - 1) / kScanThreads;
  const int64_t lo = 1 + tid * chunk, hi = imin(n + 1, lo + chunk);
  int64_t s = 0;
  for (int64_t i = lo; i < hi; ++i) s += row_ptr[i];
  sums[tid] = s;
  __syncthreads();
  for (int off = 1; off < kScanThreads; off <<= 1) {
    const int64_t v = tid >= off ? sums[tid - off] : 0;
    __syncthreads();
    sums[tid] += v;
    __syncthreads();
  }
  int64_t run = tid ? sums[tid - 1] : 0;
  for (int64_t i = lo; i < hi; ++i) {
    run += row_ptr[i];
    row_ptr[i] = run;
  }
  if (tid == 0) row_ptr[0] = 0;
}

struct TableArgs {
  const double* targets;
  const double* target_frames;  // (n_targets, 3, 2): columns e1, e2
  const double* sources;
  const double* source_frames;
  const double* source_quadrature;
  const int64_t* edge_index;    // (2, n_edges): target, source
  int64_t n_edges, n_targets, n_sources;
  int K;
  double* log_coordinates;   // (E, 2)
  double* distances;         // (E)
  double* polar;             // (E)
  double* transport;         // (E)
  double* quadrature;        // (E)
  double* angular_phases;    // (E, K + 1, 2)
  double* transport_phases;  // (E, K + 1, 2)
};

// One edge's tables.  Phase entries go through put(table, k, cos, sin): into the
// workgroup's LDS stage, or straight to HBM when the tables are too wide to stage.
template <class Put>
__device__ __forceinline__ void edge_row(const TableArgs& a, int64_t e, Put put) {
  const int64_t i = a.edge_index[e], j = a.edge_index[a.n_edges + e];
  if (i < 0 || i >= a.n_targets || j < 0 || j >= a.n_sources) {  // an index out of range marks its row
    const double nan = __builtin_nan("");
    reinterpret_cast<double2*>(a.log_coordinates)[e] = make_double2(nan, nan);
    a.distances[e] = a.polar[e] = a.transport[e] = a.quadrature[e] = nan;
    for (int k = 0; k <= a.K; ++k) {
      put(0, k, nan, nan);
      put(1, k, nan, nan);
    }
    return;
  }
  const double p[3] = {a.targets[3 * i], a.targets[3 * i + 1], a.targets[3 * i + 2]};
  const double q[3] = {a.sources[3 * j], a.sources[3 * j + 1], a.sources[3 * j + 2]};
  const double dot = clamp_unit(dot3(p, q));
  double c[3];
  cross3(p, q, c);
  const double d = atan2(norm3(c), dot);
  const double inv_density = d == 0.0 ? 1.0 : d / sin(d);  // r / sin r
  double ambient[3];
  for (int k = 0; k < 3; ++k) ambient[k] = inv_density * (q[k] - dot * p[k]);
  const double* ft = a.target_frames + 6 * i;
  const double* fs = a.source_frames + 6 * j;
  const double l0 = ft[0] * ambient[0] + ft[2] * ambient[1] + ft[4] * ambient[2];
  const double l1 = ft[1] * ambient[0] + ft[3] * ambient[1] + ft[5] * ambient[2];
  // R = I + K + K^2 / (1 + <q, p>), K the cross-product matrix of w = q x p = -(p x q),
  // applied to the source frame's e1; the target frame's components give the angle.
  const double w[3] = {-c[0], -c[1], -c[2]};
  const double u[3] = {fs[0], fs[2], fs[4]};
  double ku[3], kku[3];
  cross3(w, u, ku);
  cross3(w, ku, kku);
  const double inv1 = 1.0 / (1.0 + dot);
  double ru[3];
  for (int k = 0; k < 3; ++k) ru[k] = u[k] + ku[k] + kku[k] * inv1;
  const double t00 = ft[0] * ru[0] + ft[2] * ru[1] + ft[4] * ru[2];
  const double t10 = ft[1] * ru[0] + ft[3] * ru[1] + ft[5] * ru[2];
  const double gamma = atan2(t10, t00);
  const double phi = atan2(l1, l0);
  reinterpret_cast<double2*>(a.log_coordinates)[e] = make_double2(l0, l1);
  a.distances[e] = d;
  a.polar[e] = phi;
  a.transport[e] = gamma;
  a.quadrature[e] = a.source_quadrature[j] * inv_density;
  for (int k = 0; k <= a.K; ++k) {
    double sn, cs;
    sincos(phi * (double)k, &sn, &cs);
    put(0, k, cs, sn);
    sincos(gamma * (double)k, &sn, &cs);
    put(1, k, cs, sn);
  }
}

// Workgroups walk tiles of kTableThreads edges.  With the phase tables staged
// (dynamic LDS of 2 * kTableThreads * (K + 1) double2), a tile's rows of both
// tables, contiguous in HBM, leave in consecutive 16-byte stores.
__global__ __launch_bounds__(kTableThreads) void geo_tables_kernel(TableArgs a, int staged) {
  extern __shared__ double2 stage[];
  const int orders = a.K + 1;
  const int64_t n_tiles = (a.n_edges + kTableThreads - 1) / kTableThreads;
  double2* angular = reinterpret_cast<double2*>(a.angular_phases);
  double2* transport = reinterpret_cast<double2*>(a.transport_phases);
  for (int64_t tile = blockIdx.x; tile < n_tiles; tile += gridDim.x) {
    const int64_t e0 = tile * kTableThreads;
    const int64_t e = e0 + threadIdx.x;
    const int count = (int)imin(kTableThreads, a.n_edges - e0);
    if (e < a.n_edges) {
      if (staged) {
        double2* row0 = stage + threadIdx.x * orders;
        double2* row1 = stage + (kTableThreads + threadIdx.x) * orders;
        edge_row(a, e, [&](int table, int k, double cs, double sn) {
          (table ? row1 : row0)[k] = make_double2(cs, sn);
        });
      } else {
        edge_row(a, e, [&](int table, int k, double cs, double sn) {
          (table ? transport : angular)[e * orders + k] = make_double2(cs, sn);
        });
      }
    }
    if (staged) {
      __syncthreads();
      const int total = count * orders;
      for (int x = threadIdx.x; x < total; x += kTableThreads) {
        angular[e0 * orders + x] = stage[x];
        transport[e0 * orders + x] = stage[kTableThreads * orders + x];
      }
      __syncthreads();
    }
  }
}

__global__ __launch_bounds__(kTableThreads) void geo_distances_kernel(const double* __restrict__ targets,
                                                                      const double* __restrict__ sources,
                                                                      const int64_t* __restrict__ edge_index,
                                                                      int64_t n_edges, int64_t n_targets,
                                                                      int64_t n_sources, double* __restrict__ out) {
  const int64_t stride = (int64_t)gridDim.x * kTableThreads;
  for (int64_t e = (int64_t)blockIdx.x * kTableThreads + threadIdx.x; e < n_edges; e += stride) {
    const int64_t i = edge_index[e], j = edge_index[n_edges + e];
    if (i < 0 || i >= n_targets || j < 0 || j >= n_sources) {
      out[e] = __builtin_nan("");
      continue;
    }
    const double p[3] = {targets[3 * i], targets[3 * i + 1], targets[3 * i + 2]};
    const double q[3] = {sources[3 * j], sources[3 * j + 1], sources[3 * j + 2]};
    out[e] = geodesic(p, q, dot3(p, q));
  }
}

int64_t tiles_of(int64_t n) { return (n + kGeoTile - 1) / kGeoTile; }

int64_t table_blocks(int64_t n_edges) {
  return std::max<int64_t>(1, std::min<int64_t>((n_edges + kTableThreads - 1) / kTableThreads, 8192));
}

int prepare_walk(WalkArgs& a, const double* targets, int64_t n_targets, const double* sources, int64_t n_sources,
                 double limit, const double* workspace) {
  GM_REQUIRE(n_targets >= 1 && n_sources >= 1, "the target and source node sets must be non-empty");
  GM_REQUIRE(tiles_of(n_targets) <= INT32_MAX, "too many target nodes for one launch");
  GM_REQUIRE(targets && sources && workspace && aligned(targets, 8) && aligned(sources, 8) && aligned(workspace, 8),
             "targets, sources and workspace must be 8-byte aligned device pointers");
  GM_REQUIRE(std::isfinite(limit) && limit > 0.0, "the radius limit must be positive and finite");
  a.targets = targets;
  a.sources = sources;
  a.target_boxes = workspace;
  a.source_boxes = workspace + 6 * tiles_of(n_targets);
  a.n_targets = n_targets;
  a.n_sources = n_sources;
  a.limit = limit;
  const double pi = 3.14159265358979323846;
  // The computed <p, q> of unit vectors is within ~1e-15 of cos(angle) and |d cos| <= |d angle|:
  // 1e-12 on either side of cos(limit) bounds the band where only the exact test decides.
  a.cos_floor = limit >= pi ? -2.0 : std::cos(limit) - 1e-12;
  a.cos_in = limit >= pi ? -2.0 : std::cos(limit) + 1e-12;
  a.reach = (limit >= pi ? 2.0 : 2.0 * std::sin(0.5 * limit)) + 1e-9;
  return GM_OK;
}

}  // namespace
}  // namespace gm

extern "C" int64_t gm_radius_workspace_doubles(int64_t n_targets, int64_t n_sources) {
  return 6 * (gm::tiles_of(n_targets) + gm::tiles_of(n_sources));
}

extern "C" int gm_radius_row_ptr_f64(const double* targets, int64_t n_targets, const double* sources,
                                     int64_t n_sources, double limit, double* workspace, int64_t* row_ptr,
                                     void* stream) {
  gm::WalkArgs a{};
  const int status = gm::prepare_walk(a, targets, n_targets, sources, n_sources, limit, workspace);
  if (status != GM_OK) return status;
  GM_REQUIRE(row_ptr && gm::aligned(row_ptr, 8), "row_ptr must be an 8-byte aligned device pointer");
  a.row_ptr = row_ptr;
  const hipStream_t s = (hipStream_t)stream;
  const int64_t tt = gm::tiles_of(n_targets), ts = gm::tiles_of(n_sources);
  hipLaunchKernelGGL(gm::geo_bounds_kernel, dim3(tt), dim3(gm::kGeoTile), 0, s, targets, n_targets, workspace);
  hipLaunchKernelGGL(gm::geo_bounds_kernel, dim3(ts), dim3(gm::kGeoTile), 0, s, sources, n_sources,
                     workspace + 6 * tt);
  int rc = gm::check_launch("radius_bounds");
  if (rc != GM_OK) return rc;
  hipLaunchKernelGGL(gm::geo_walk_kernel<false>, dim3(tt), dim3(gm::kGeoTile), 0, s, a);
  rc = gm::check_launch("radius_degrees");
  if (rc != GM_OK) return rc;
  hipLaunchKernelGGL(gm::geo_scan_kernel, dim3(1), dim3(gm::kScanThreads), 0, s, row_ptr, n_targets);
  return gm::check_launch("radius_row_ptr");
}

extern "C" int gm_radius_edges_f64(const double* targets, int64_t n_targets, const double* sources,
                                   int64_t n_sources, double limit, const double* workspace, const int64_t* row_ptr,
                                   int64_t n_edges, int64_t* edge_index, void* stream) {
  gm::WalkArgs a{};
  const int status = gm::prepare_walk(a, targets, n_targets, sources, n_sources, limit, workspace);
  if (status != GM_OK) return status;
  GM_REQUIRE(row_ptr && gm::aligned(row_ptr, 8), "row_ptr must be an 8-byte aligned device pointer");
  GM_REQUIRE(n_edges >= 0, "n_edges must be non-negative");
  if (n_edges == 0) return GM_OK;
  GM_REQUIRE(edge_index && gm::aligned(edge_index, 8), "edge_index must be an 8-byte aligned device pointer");
  a.row_ptr = const_cast<int64_t*>(row_ptr);
  a.target_out = edge_index;
  a.source_out = edge_index + n_edges;
  a.n_edges = n_edges;
  hipLaunchKernelGGL(gm::geo_walk_kernel<true>, dim3(gm::tiles_of(n_targets)), dim3(gm::kGeoTile), 0,
                     (hipStream_t)stream, a);
  return gm::check_launch("radius_edges");
}

extern "C" int gm_geodesic_distances_f64(const double* targets, const double* sources, const int64_t* edge_index,
                                         int64_t n_edges, int64_t n_targets, int64_t n_sources, double* distances,
                                         void* stream) {
  GM_REQUIRE(n_edges >= 0 && n_targets >= 0 && n_sources >= 0, "counts must be non-negative");
  if (n_edges == 0) return GM_OK;
  GM_REQUIRE(targets && sources && edge_index && distances, "every pointer must be a device pointer");
  hipLaunchKernelGGL(gm::geo_distances_kernel, dim3(gm::table_blocks(n_edges)), dim3(gm::kTableThreads), 0,
                     (hipStream_t)stream, targets, sources, edge_index, n_edges, n_targets, n_sources, distances);
  return gm::check_launch("geodesic_distances");
}

extern "C" int gm_edge_tables_f64(const double* targets, const double* target_frames, const double* sources,
                                  const double* source_frames, const double* source_quadrature,
                                  const int64_t* edge_index, int64_t n_edges, int64_t n_targets, int64_t n_sources,
                                  int64_t max_frequency, double* log_coordinates, double* distances,
                                  double* polar_angles, double* transport_angles, double* tangent_quadrature,
                                  double* angular_phases, double* transport_phases, void* stream) {
  GM_REQUIRE(n_edges >= 0 && n_targets >= 0 && n_sources >= 0, "counts must be non-negative");
  GM_REQUIRE(max_frequency >= 0 && max_frequency <= 64, "max_frequency must lie in [0, 64]");
  if (n_edges == 0) return GM_OK;
  GM_REQUIRE(targets && target_frames && sources && source_frames && source_quadrature && edge_index,
             "node, frame, quadrature and edge pointers must be device pointers");
  GM_REQUIRE(log_coordinates && distances && polar_angles && transport_angles && tangent_quadrature &&
                 angular_phases && transport_phases,
             "every output must be a device pointer");
  GM_REQUIRE(gm::aligned(log_coordinates, 16) && gm::aligned(angular_phases, 16) && gm::aligned(transport_phases, 16),
             "log_coordinates and the phase tables must be 16-byte aligned");
  gm::TableArgs a{};
  a.targets = targets;
  a.target_frames = target_frames;
  a.sources = sources;
  a.source_frames = source_frames;
  a.source_quadrature = source_quadrature;
  a.edge_index = edge_index;
  a.n_edges = n_edges;
  a.n_targets = n_targets;
  a.n_sources = n_sources;
  a.K = (int)max_frequency;
  a.log_coordinates = log_coordinates;
  a.distances = distances;
  a.polar = polar_angles;
  a.transport = transport_angles;
  a.quadrature = tangent_quadrature;
  a.angular_phases = angular_phases;
  a.transport_phases = transport_phases;
  // Stage the phase tables through LDS while they fit four workgroups per CU.
  const size_t stage_bytes = 2 * gm::kTableThreads * (size_t)(max_frequency + 1) * sizeof(double2);
  const int staged = stage_bytes <= 40 * 1024;
  hipLaunchKernelGGL(gm::geo_tables_kernel, dim3(gm::table_blocks(n_edges)), dim3(gm::kTableThreads),
                     staged ? stage_bytes : 0, (hipStream_t)stream, a, staged);
  return gm::check_launch("edge_tables");
}
