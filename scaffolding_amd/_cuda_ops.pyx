# cython: language_level=3, cdivision=True
"""
_cuda_ops — the operator seam of the matmul hot path, MI355X edition.

Exports the Python names Scaffolding's tensor / nn layers import as
``_cuops`` (reference seam: /root/reference/_cuda_ops.pyx; importers listed
at tensor.py:36-41, nn/layers.py:12, nn/functional.py:11).  Every compute
entry point calls libsfgemm's C ABI (include/sfgemm.h) on the HIP device;
nothing here computes on the host.  There is no fallback: without the
library this module does not import, and without a GPU every device call
raises RuntimeError.

Differences from the reference, on purpose:
  * real 16-bit storage: GpuTensor.dtype may be np.float16 or BFLOAT16 (a
    2-byte structured dtype standing for bfloat16); GEMM outputs keep the
    input dtype, as np.matmul does, instead of always being tagged fp32
    (reference _cuda_ops.pyx:1102,1149,1302);
  * dev_linear_forward takes an optional fused activation ('silu' or
    'gelu'), and dev_batched_matmul_nt / dev_matmul_nt an alpha, so bias,
    activation and the SDPA scale are GEMM epilogues, not extra passes;
  * batched matmul broadcasts a 2-D operand over the other's batch, as
    np.matmul does (the reference assumes equal batch, :1122-1149);
  * dev_softmax over a non-last dim raises instead of silently using the
    last dim (reference :1016-1034 ignores `dim`).
"""

import numpy as np
cimport numpy as cnp
from libc.stdint cimport int64_t, uint64_t, uintptr_t
from libc.string cimport memset
from libc.math cimport sqrt

cnp.import_array()

cdef extern from "sfgemm.h" nogil:
    ctypedef enum sf_dtype:
        SF_F32
        SF_F16
        SF_BF16
    ctypedef enum sf_epilogue:
        SF_EPI_NONE
        SF_EPI_BIAS
        SF_EPI_BIAS_SILU
        SF_EPI_BIAS_GELU_TANH
        SF_EPI_SILU
        SF_EPI_GELU_TANH
    int SF_OK
    int SF_ERR_HIP
    int SF_ERR_INVALID_ARG
    int SF_ERR_UNSUPPORTED
    int SF_ERR_NO_DEVICE
    int SF_ERR_OOM

    const char* sf_status_string(int status)
    const char* sf_last_error()
    int sf_version()
    int sf_set_test_hooks(int xcd_shift, int split_spins, int attn_parts)

    int sf_gemm(int transA, int transB, int64_t M, int64_t N, int64_t K, int64_t batch,
                const void* A, int64_t lda, int64_t strideA,
                const void* B, int64_t ldb, int64_t strideB,
                void* C, int64_t ldc, int64_t strideC,
                sf_dtype ab_dtype, sf_dtype c_dtype, float alpha,
                const void* bias, sf_epilogue epi, void* stream)
    int sf_gemm_plan(int transA, int transB, int64_t M, int64_t N, int64_t K, int64_t batch,
                     const void* A, int64_t lda, int64_t strideA,
                     const void* B, int64_t ldb, int64_t strideB,
                     void* C, int64_t ldc, int64_t strideC,
                     sf_dtype ab_dtype, sf_dtype c_dtype, float alpha,
                     const void* bias, sf_epilogue epi, char* buf, int len)
    int sf_attention(const void* Q, int64_t ldq, int64_t strideQ,
                     const void* K, int64_t ldk, int64_t strideK,
                     const void* V, int64_t ldv, int64_t strideV,
                     void* O, int64_t ldo, int64_t strideO,
                     int64_t batch, int64_t Sq, int64_t Sk, int64_t D,
                     float scale, sf_dtype dtype, void* stream)
    int sf_gemm_add(int transA, int transB, int64_t M, int64_t N, int64_t K, int64_t batch,
                    const void* A, int64_t lda, int64_t strideA,
                    const void* B, int64_t ldb, int64_t strideB,
                    void* C, int64_t ldc, int64_t strideC,
                    sf_dtype ab_dtype, sf_dtype c_dtype, float alpha,
                    const void* bias, sf_epilogue epi,
                    const void* R, int64_t ldr, int64_t strideR, void* stream)
    int sf_attention_heads(const void* Q, int64_t ldq, int64_t strideQ, int64_t headQ,
                           const void* K, int64_t ldk, int64_t strideK, int64_t headK,
                           const void* V, int64_t ldv, int64_t strideV, int64_t headV,
                           void* O, int64_t ldo, int64_t strideO, int64_t headO,
                           int64_t batch, int64_t heads, int64_t Sq, int64_t Sk, int64_t D,
                           float scale, sf_dtype dtype, void* stream)
    int sf_layer_norm(const void* x, void* y, int64_t rows, int64_t cols,
                      const void* gamma, const void* beta, float eps,
                      const void* mod_scale, const void* mod_shift, int64_t mod_ld, int64_t group_rows,
                      float* mean_out, float* rstd_out, sf_dtype dt, void* stream)
    int sf_rms_norm(const void* x, void* y, int64_t rows, int64_t cols,
                    const void* gamma, float eps, sf_dtype dt, void* stream)
    int sf_add(const void* a, const void* b, void* y, int64_t n, sf_dtype dt, void* stream)
    int sf_softmax_rows(const void* x, void* y, int64_t rows, int64_t cols,
                        sf_dtype in_dtype, sf_dtype out_dtype, float scale, void* stream)
    int sf_softmax_rows_masked(const void* x, void* y, int64_t rows, int64_t cols,
                               sf_dtype dtype, float scale, const void* mask, sf_dtype mask_dtype,
                               int64_t rows_per_batch, int64_t inner_batches,
                               int64_t stride_outer, int64_t stride_inner,
                               int64_t stride_row, int64_t stride_col, void* stream)
    int sf_silu(const void* x, void* y, int64_t n, sf_dtype dt, void* stream)
    int sf_gelu(const void* x, void* y, int64_t n, sf_dtype dt, void* stream)
    int sf_muls(const void* x, float s, void* y, int64_t n, sf_dtype dt, void* stream)
    int sf_bias_add_rows(void* C, const void* bias, int64_t M, int64_t N, sf_dtype dt, void* stream)
    int sf_dropout(const void* x, void* y, void* mask, int64_t n, sf_dtype dt, float p, uint64_t seed,
                   uint64_t offset, void* stream)
    int sf_sum_dim(const void* x, void* out, int64_t outer, int64_t dim_size, int64_t inner,
                   sf_dtype in_dtype, sf_dtype out_dtype, void* stream)
    int sf_cast(const void* x, sf_dtype in_dtype, void* y, sf_dtype out_dtype, int64_t n, void* stream)

    int sf_get_device_count(int* count)
    int sf_set_device(int device)
    int sf_get_device(int* device)
    int sf_device_synchronize()
    int sf_get_device_name(int device, char* buf, int len)
    int sf_get_device_arch(int device, char* buf, int len)
    int sf_get_device_props(int device, int* cu_count, int64_t* total_mem, int* clock_khz, int* l2_bytes)
    int sf_mem_get_info(size_t* free_bytes, size_t* total_bytes)
    int sf_cache_alloc(int device, size_t nbytes, void** ptr, size_t* got_bytes)
    int sf_cache_free(int device, void* ptr, size_t nbytes)
    int sf_cache_empty(int device)
    int sf_cache_stats(int device, size_t* pooled_bytes, size_t* live_bytes)
    int sf_cache_set_limit(size_t bytes_per_device)
    int sf_memcpy_h2d(void* dst, const void* src, size_t nbytes, void* stream)
    int sf_memcpy_d2h(void* dst, const void* src, size_t nbytes, void* stream)
    int sf_memcpy_d2d(void* dst, const void* src, size_t nbytes, void* stream)
    int sf_zero(void* dst, size_t nbytes, void* stream)
    int sf_stream_create(void** stream)
    int sf_stream_destroy(void* stream)
    int sf_stream_synchronize(void* stream)
    int sf_event_create(void** event)
    int sf_event_destroy(void* event)
    int sf_event_record(void* event, void* stream)
    int sf_event_synchronize(void* event)
    int sf_stream_wait_event(void* stream, void* event)
    int sf_event_elapsed_ms(float* ms, void* start, void* end)


# ================================================================
#  dtypes
# ================================================================

# bfloat16 storage dtype: 2 bytes, distinct from np.uint16 so it can never
# be mistaken for integer data.  Host views of device bfloat16 data are
# widened to float32 (the reference's own host mapping, dtype.py:31).
BFLOAT16 = np.dtype([('bf16', '<u2')])

_F32 = np.dtype(np.float32)
_F16 = np.dtype(np.float16)


cdef sf_dtype _sf_dtype(object dt) except *:
    d = np.dtype(dt) if not isinstance(dt, np.dtype) else dt
    if d == _F32:
        return SF_F32
    if d == _F16:
        return SF_F16
    if d == BFLOAT16:
        return SF_BF16
    raise TypeError("unsupported device dtype %r (float32, float16, bfloat16 only)" % (dt,))


cdef size_t _itemsize(object dt) except 0:
    return (<object>np.dtype(dt)).itemsize


def resolve_dtype(dt):
    """Maps 'bfloat16' / 'float16' / 'float32' / numpy dtypes to the device
    storage dtype used in GpuTensor.dtype."""
    if isinstance(dt, str):
        if dt in ('bfloat16', 'bf16'):
            return BFLOAT16
        return np.dtype(dt)
    if isinstance(dt, np.dtype):
        return dt
    return np.dtype(dt)


# ================================================================
#  Errors (text as the reference's _cuda_ops.pyx:292-300)
# ================================================================

cdef inline str _detail(int ret):
    cdef const char* d = sf_last_error()
    msg = d.decode('utf-8', 'replace') if d != NULL else ''
    if not msg:
        msg = sf_status_string(ret).decode('utf-8')
    return msg


cdef inline void _check_cuda(int ret) except *:
    if ret != SF_OK:
        raise RuntimeError("CUDA error: %s" % _detail(ret))


cdef inline void _check_kernel(int ret) except *:
    if ret != SF_OK:
        raise RuntimeError("CUDA kernel launch failed with ret code %d: %s" % (ret, _detail(ret)))


# ================================================================
#  Device buffer (reference CudaBuffer, _cuda_ops.pyx:307-341)
# ================================================================

cdef class CudaBuffer:
    """Owning handle of device memory from the native caching allocator;
    returned to the pool when the Python object dies."""
    cdef void* ptr
    cdef size_t nbytes
    cdef int device_id
    cdef bint owns_memory

    def __cinit__(self):
        self.ptr = NULL
        self.nbytes = 0
        self.device_id = 0
        self.owns_memory = False

    def __dealloc__(self):
        if self.owns_memory and self.ptr != NULL:
            sf_cache_free(self.device_id, self.ptr, self.nbytes)
            self.ptr = NULL

    @property
    def data_ptr(self):
        return <uintptr_t>self.ptr

    @property
    def size(self):
        return self.nbytes

    @property
    def device(self):
        return self.device_id


cdef CudaBuffer _make_buffer(size_t nbytes, int device_id):
    cdef CudaBuffer buf = CudaBuffer.__new__(CudaBuffer)
    cdef size_t got = 0
    cdef void* p = NULL
    cdef int ret
    with nogil:
        ret = sf_cache_alloc(device_id, nbytes, &p, &got)
    _check_cuda(ret)
    buf.ptr = p
    buf.nbytes = got
    buf.device_id = device_id
    buf.owns_memory = True
    return buf


cdef int _current_device() except -1:
    cdef int dev = 0
    _check_cuda(sf_get_device(&dev))
    return dev


def empty_cache(int device=-1):
    """Frees every pooled (unused) device block (reference :413-437)."""
    _check_cuda(sf_cache_empty(device))


def cache_stats(int device=-1):
    """(pooled_bytes, live_bytes) of the native caching allocator."""
    cdef size_t pooled = 0, live = 0
    sf_cache_stats(device, &pooled, &live)
    return int(pooled), int(live)


def set_cache_limit(size_t nbytes):
    sf_cache_set_limit(nbytes)


# ================================================================
#  GpuTensor (reference _cuda_ops.pyx:807-819)
# ================================================================

class GpuTensor:
    """GPU-resident, C-contiguous tensor: a CudaBuffer plus shape and dtype."""
    __slots__ = ('buffer', 'shape', 'dtype', 'numel', 'device_id')

    def __init__(self, buffer, tuple shape, dtype, int device_id=-1):
        self.buffer = buffer
        self.shape = tuple(int(s) for s in shape)
        self.dtype = resolve_dtype(dtype)
        self.device_id = device_id if device_id >= 0 else (<CudaBuffer>buffer).device_id
        cdef int64_t n = 1
        for s in self.shape:
            n *= s
        self.numel = n

    @property
    def nbytes(self):
        return self.numel * self.dtype.itemsize

    @property
    def data_ptr(self):
        return (<CudaBuffer>self.buffer).data_ptr

    def __repr__(self):
        name = 'bfloat16' if self.dtype == BFLOAT16 else str(self.dtype)
        return "GpuTensor(shape=%s, dtype=%s, device=%d)" % (self.shape, name, self.device_id)


cdef inline void* _ptr(gt) except? NULL:
    return (<CudaBuffer>(gt.buffer)).ptr


cdef object _alloc_like(tuple shape, dtype, int device_id):
    cdef int64_t n = 1
    for s in shape:
        n *= s
    cdef size_t nbytes = <size_t>n * _itemsize(dtype)
    return GpuTensor(_make_buffer(nbytes, device_id), shape, dtype, device_id)


def empty(tuple shape, dtype=np.float32, int device_id=-1):
    """Uninitialised device tensor."""
    if device_id < 0:
        device_id = _current_device()
    return _alloc_like(shape, resolve_dtype(dtype), device_id)


def zeros(tuple shape, dtype=np.float32, int device_id=-1):
    gt = empty(shape, dtype, device_id)
    cdef size_t nb = gt.nbytes
    _check_kernel(sf_zero(_ptr(gt), nb, NULL))
    return gt


def gputensor_from_numpy(cnp.ndarray arr not None, int device_id=-1, dtype=None):
    """Uploads a NumPy array (reference :822-840).  dtype='bfloat16' (or
    BFLOAT16) uploads float32 data and rounds it to bfloat16 on the device
    (RNE); dtype=np.float16 likewise from float32 input."""
    cdef int target = device_id
    cdef int prev = 0
    if target < 0:
        target = _current_device()
    target_dt = resolve_dtype(dtype) if dtype is not None else arr.dtype
    if target_dt == BFLOAT16 and arr.dtype == BFLOAT16:
        src = np.ascontiguousarray(arr)
        host_dt = BFLOAT16
    elif target_dt == BFLOAT16 or (dtype is not None and target_dt != arr.dtype):
        src = np.ascontiguousarray(arr, dtype=np.float32)
        host_dt = _F32
    else:
        src = np.ascontiguousarray(arr)
        host_dt = src.dtype
    if host_dt != BFLOAT16 and host_dt not in (_F32, _F16):
        raise TypeError("gputensor_from_numpy: unsupported dtype %r" % (arr.dtype,))
    cdef cnp.ndarray flat = src.reshape(-1)
    cdef size_t nbytes = flat.nbytes
    shape = tuple((<object>arr).shape)
    staged = _alloc_like(shape, host_dt, target)
    _check_cuda(sf_get_device(&prev))
    if prev != target:
        _check_cuda(sf_set_device(target))
    try:
        _check_cuda(sf_memcpy_h2d(_ptr(staged), cnp.PyArray_DATA(flat), nbytes, NULL))
        if host_dt == target_dt:
            return staged
        out = _alloc_like(shape, target_dt, target)
        _check_kernel(sf_cast(_ptr(staged), _sf_dtype(host_dt), _ptr(out), _sf_dtype(target_dt),
                              staged.numel, NULL))
        return out
    finally:
        if prev != target:
            sf_set_device(prev)


def gputensor_to_numpy(gt):
    """Downloads a GpuTensor (reference :843-858).  bfloat16 data comes back
    widened to float32 (exact)."""
    cdef int prev = 0
    cdef int tgt = gt.device_id
    cdef cnp.ndarray result
    _check_cuda(sf_get_device(&prev))
    if prev != tgt:
        _check_cuda(sf_set_device(tgt))
    try:
        src = gt
        if gt.dtype == BFLOAT16:
            src = _alloc_like(gt.shape, _F32, tgt)
            _check_kernel(sf_cast(_ptr(gt), SF_BF16, _ptr(src), SF_F32, gt.numel, NULL))
        result = np.empty(src.shape, dtype=src.dtype)
        _check_cuda(sf_memcpy_d2h(cnp.PyArray_DATA(result), _ptr(src), <size_t>result.nbytes, NULL))
        return result
    finally:
        if prev != tgt:
            sf_set_device(prev)


def gputensor_bits_to_numpy(gt):
    """Raw storage download: bfloat16 as uint16 bit patterns."""
    cdef cnp.ndarray result
    dt = np.dtype(np.uint16) if gt.dtype == BFLOAT16 else gt.dtype
    result = np.empty(gt.shape, dtype=dt)
    _check_cuda(sf_memcpy_d2h(cnp.PyArray_DATA(result), _ptr(gt), <size_t>result.nbytes, NULL))
    return result


def gputensor_from_bits(cnp.ndarray bits not None, int device_id=-1):
    """Uploads uint16 bfloat16 bit patterns as a bfloat16 GpuTensor."""
    if bits.dtype != np.uint16:
        raise TypeError("gputensor_from_bits expects uint16 bit patterns")
    return gputensor_from_numpy(np.ascontiguousarray(bits).view(BFLOAT16), device_id)


def gputensor_to_device(gt, int target_dev):
    """Copies a GpuTensor to another device (reference :861-875)."""
    if gt.device_id == target_dev:
        return gt
    out = _alloc_like(gt.shape, gt.dtype, target_dev)
    _check_cuda(sf_memcpy_d2d(_ptr(out), _ptr(gt), <size_t>gt.nbytes, NULL))
    _check_cuda(sf_device_synchronize())
    return out


def dev_copy(gt_src, gt_dst):
    """Copies src's bytes into dst on the device (reference :1354-1364):
    equal element counts and dtypes, asynchronous on the default stream."""
    if gt_src.numel != gt_dst.numel or gt_src.dtype != gt_dst.dtype:
        raise ValueError("dev_copy: %s %s into %s %s" % (gt_src.shape, gt_src.dtype, gt_dst.shape, gt_dst.dtype))
    if gt_src.numel == 0:
        return gt_dst
    _check_cuda(sf_memcpy_d2d(_ptr(gt_dst), _ptr(gt_src), <size_t>gt_src.nbytes, NULL))
    return gt_dst


def dev_cast(gt, dtype):
    """Device dtype conversion (RNE)."""
    dt = resolve_dtype(dtype)
    if dt == gt.dtype:
        return gt
    out = _alloc_like(gt.shape, dt, gt.device_id)
    _check_kernel(sf_cast(_ptr(gt), _sf_dtype(gt.dtype), _ptr(out), _sf_dtype(dt), gt.numel, NULL))
    return out


def dev_reshape(gt, tuple shape):
    """Metadata-only view (reference :1397-1420)."""
    cdef int64_t n = 1
    for s in shape:
        n *= s
    if n != gt.numel:
        raise ValueError("cannot reshape %s into %s" % (gt.shape, shape))
    return GpuTensor(gt.buffer, shape, gt.dtype, gt.device_id)


# ================================================================
#  Devices, streams, events (reference :491-685)
# ================================================================

def get_device_count():
    cdef int n = 0
    if sf_get_device_count(&n) != SF_OK:
        return 0
    return n


def set_device(int device):
    _check_cuda(sf_set_device(device))


def get_current_device():
    return _current_device()


def device_synchronize():
    cdef int ret
    with nogil:
        ret = sf_device_synchronize()
    _check_cuda(ret)


def get_device_name(int device=0):
    cdef char buf[256]
    _check_cuda(sf_get_device_name(device, buf, 256))
    return buf.decode('utf-8', 'replace')


def get_device_arch(int device=0):
    cdef char buf[256]
    _check_cuda(sf_get_device_arch(device, buf, 256))
    return buf.decode('utf-8', 'replace')


def get_device_properties(int device):
    cdef int cus = 0, clk = 0, l2 = 0
    cdef int64_t mem = 0
    _check_cuda(sf_get_device_props(device, &cus, &mem, &clk, &l2))
    return {
        'name': get_device_name(device),
        'arch': get_device_arch(device),
        'total_memory': int(mem),
        'multi_processor_count': cus,
        'clock_rate_khz': clk,
        'l2_cache_size': l2,
    }


def get_device_capability(int device=0):
    """(9, 5) for gfx950."""
    arch = get_device_arch(device).split(':')[0]
    digits = arch[3:] if arch.startswith('gfx') else ''
    if len(digits) >= 3:
        return (int(digits[:-2]), int(digits[-2:-1], 16))
    return (0, 0)


def mem_info():
    cdef size_t f = 0, t = 0
    _check_cuda(sf_mem_get_info(&f, &t))
    return int(f), int(t)


def set_tf32_enabled(bint enable):
    """Accepted and ignored (reference :2474): the fp32 path always runs
    true fp32 MFMA; gfx950 has no reduced-precision fp32 matrix mode."""
    return None


cdef class CudaStream:
    """HIP stream at default priority (reference :608-665)."""
    cdef void* stream
    cdef int _device_id

    def __cinit__(self, int device_id=0, bint non_blocking=True):
        self.stream = NULL
        self._device_id = device_id
        _check_cuda(sf_stream_create(&self.stream))

    def __dealloc__(self):
        if self.stream != NULL:
            sf_stream_destroy(self.stream)
            self.stream = NULL

    def synchronize(self):
        _check_cuda(sf_stream_synchronize(self.stream))

    def wait_event(self, CudaEvent event):
        _check_cuda(sf_stream_wait_event(self.stream, event.event))

    @property
    def cuda_stream(self):
        return <uintptr_t>self.stream

    @property
    def device_id(self):
        return self._device_id


cdef class CudaEvent:
    """HIP event with timing (reference :646-673)."""
    cdef void* event

    def __cinit__(self, bint enable_timing=True):
        self.event = NULL
        _check_cuda(sf_event_create(&self.event))

    def __dealloc__(self):
        if self.event != NULL:
            sf_event_destroy(self.event)
            self.event = NULL

    def record(self, stream=None):
        cdef void* s = NULL
        if stream is not None:
            s = <void*><uintptr_t>(stream.cuda_stream)
        _check_cuda(sf_event_record(self.event, s))

    def synchronize(self):
        _check_cuda(sf_event_synchronize(self.event))

    def elapsed_time(self, CudaEvent end):
        cdef float ms = 0
        _check_cuda(sf_event_elapsed_ms(&ms, self.event, end.event))
        return ms


# ================================================================
#  GEMM family (reference :1088-1190, :1278-1302)
# ================================================================

cdef object _same_dtype(a, b, str name):
    if a.dtype != b.dtype:
        raise TypeError("%s: operand dtypes differ (%s vs %s)" % (name, a.dtype, b.dtype))
    return a.dtype


cdef object _gemm(int transB, int64_t M, int64_t N, int64_t K, int64_t batch,
                  a, int64_t strideA, b, int64_t ldb, int64_t strideB,
                  tuple out_shape, float alpha, bias, int epi, residual=None):
    dt = a.dtype
    cdef sf_dtype sdt = _sf_dtype(dt)
    cdef int dev = a.device_id
    out = _alloc_like(out_shape, dt, dev)
    cdef void* pa = _ptr(a)
    cdef void* pb = _ptr(b)
    cdef void* pc = _ptr(out)
    cdef void* pbias = NULL
    cdef void* pr = NULL
    if bias is not None:
        pbias = _ptr(bias)
    if residual is not None:
        pr = _ptr(residual)
    cdef int ret
    cdef int64_t lda = K if K > 0 else 1
    if transB and ldb < 1:
        ldb = 1
    with nogil:
        if pr != NULL:
            ret = sf_gemm_add(0, transB, M, N, K, batch, pa, lda, strideA, pb, ldb, strideB,
                              pc, N, M * N, sdt, sdt, alpha, pbias, <sf_epilogue>epi, pr, N, M * N, NULL)
        else:
            ret = sf_gemm(0, transB, M, N, K, batch, pa, lda, strideA, pb, ldb, strideB,
                          pc, N, M * N, sdt, sdt, alpha, pbias, <sf_epilogue>epi, NULL)
    _check_kernel(ret)
    return out


cdef object _gemm_tn(int64_t M, int64_t N, int64_t K, int64_t batch, a, int64_t strideA, b,
                     int64_t strideB, tuple out_shape, float alpha):
    """C = alpha * A^T . B with A stored K x M and B stored K x N."""
    dt = a.dtype
    cdef sf_dtype sdt = _sf_dtype(dt)
    out = _alloc_like(out_shape, dt, a.device_id)
    cdef void* pa = _ptr(a)
    cdef void* pb = _ptr(b)
    cdef void* pc = _ptr(out)
    cdef int ret
    cdef int64_t lda = M if M > 0 else 1
    cdef int64_t ldb = N if N > 0 else 1
    with nogil:
        ret = sf_gemm(1, 0, M, N, K, batch, pa, lda, strideA, pb, ldb, strideB,
                      pc, N, M * N, sdt, sdt, alpha, NULL, SF_EPI_NONE, NULL)
    _check_kernel(ret)
    return out


def gemm_plan(int transB, int64_t M, int64_t N, int64_t K, int64_t batch,
              uintptr_t ptr_a, int64_t lda, int64_t stride_a,
              uintptr_t ptr_b, int64_t ldb, int64_t stride_b,
              int64_t ldc, int64_t stride_c, dtype, out_dtype=None, int epi=0,
              uintptr_t ptr_bias=0, int transA=0):
    """Name of the kernel sf_gemm would launch for these arguments (host
    only; pointers are plain integers and are never dereferenced)."""
    cdef char buf[128]
    cdef sf_dtype ab = _sf_dtype(resolve_dtype(dtype))
    cdef sf_dtype c = _sf_dtype(resolve_dtype(out_dtype)) if out_dtype is not None else ab
    cdef int ret = sf_gemm_plan(transA, transB, M, N, K, batch, <void*>ptr_a, lda, stride_a,
                                <void*>ptr_b, ldb, stride_b, NULL, ldc, stride_c, ab, c, 1.0,
                                <void*>ptr_bias, <sf_epilogue>epi, buf, 128)
    _check_kernel(ret)
    return buf.decode('utf-8')


def dev_matmul(gt_a, gt_b):
    """C = A @ B, A (M,K), B (K,N)  (reference :1088-1102)."""
    _same_dtype(gt_a, gt_b, 'dev_matmul')
    if len(gt_a.shape) != 2 or len(gt_b.shape) != 2:
        raise ValueError("dev_matmul expects 2-D operands")
    cdef int64_t M = gt_a.shape[0], K = gt_a.shape[1], N = gt_b.shape[1]
    if gt_b.shape[0] != K:
        raise ValueError("dev_matmul: shapes %s and %s not aligned" % (gt_a.shape, gt_b.shape))
    return _gemm(0, M, N, K, 1, gt_a, 0, gt_b, N, 0, (M, N), 1.0, None, SF_EPI_NONE)


def dev_matmul_nt(gt_a, gt_b, float alpha=1.0):
    """C = alpha * A @ B^T, A (M,K), B (N,K)  (reference :1105-1119)."""
    _same_dtype(gt_a, gt_b, 'dev_matmul_nt')
    if len(gt_a.shape) != 2 or len(gt_b.shape) != 2:
        raise ValueError("dev_matmul_nt expects 2-D operands")
    cdef int64_t M = gt_a.shape[0], K = gt_a.shape[1], N = gt_b.shape[0]
    if gt_b.shape[1] != K:
        raise ValueError("dev_matmul_nt: shapes %s and %s not aligned" % (gt_a.shape, gt_b.shape))
    return _gemm(1, M, N, K, 1, gt_a, 0, gt_b, K, 0, (M, N), alpha, None, SF_EPI_NONE)


cdef tuple _batch_layout(tuple a_shape, tuple b_shape, int64_t a_mat, int64_t b_mat, str name):
    """Batch size, operand batch strides and batch shape under np.matmul's
    rule for the cases this path meets: equal batch dims, or a 2-D operand
    broadcast over the other's batch."""
    a_b = a_shape[:-2]
    b_b = b_shape[:-2]
    if a_b == b_b:
        bshape = a_b
        sa, sb = a_mat, b_mat
    elif len(b_b) == 0:
        bshape = a_b
        sa, sb = a_mat, 0
    elif len(a_b) == 0:
        bshape = b_b
        sa, sb = 0, b_mat
    else:
        raise ValueError("%s: batch dims %s and %s do not match" % (name, a_b, b_b))
    cdef int64_t batch = 1
    for s in bshape:
        batch *= s
    return batch, sa, sb, tuple(bshape)


def dev_batched_matmul(gt_a, gt_b):
    """C[...] = A[...] @ B[...], A (...,M,K), B (...,K,N)  (reference :1122-1149)."""
    _same_dtype(gt_a, gt_b, 'dev_batched_matmul')
    a_shape, b_shape = gt_a.shape, gt_b.shape
    if len(a_shape) < 2 or len(b_shape) < 2:
        raise ValueError("dev_batched_matmul expects operands of rank >= 2")
    cdef int64_t M = a_shape[-2], K = a_shape[-1], N = b_shape[-1]
    if b_shape[-2] != K:
        raise ValueError("dev_batched_matmul: shapes %s and %s not aligned" % (a_shape, b_shape))
    batch, sa, sb, bshape = _batch_layout(a_shape, b_shape, M * K, K * N, 'dev_batched_matmul')
    return _gemm(0, M, N, K, batch, gt_a, sa, gt_b, N, sb, bshape + (M, N), 1.0, None, SF_EPI_NONE)


def dev_batched_matmul_nt(gt_a, gt_b, float alpha=1.0):
    """C[...] = alpha * A[...] @ B[...]^T, A (...,M,K), B (...,N,K), one
    strided-batched launch (the reference loops over the batch in Python,
    :1152-1190)."""
    _same_dtype(gt_a, gt_b, 'dev_batched_matmul_nt')
    a_shape, b_shape = gt_a.shape, gt_b.shape
    if len(a_shape) < 2 or len(b_shape) < 2:
        raise ValueError("dev_batched_matmul_nt expects operands of rank >= 2")
    cdef int64_t M = a_shape[-2], K = a_shape[-1], N = b_shape[-2]
    if b_shape[-1] != K:
        raise ValueError("dev_batched_matmul_nt: shapes %s and %s not aligned" % (a_shape, b_shape))
    batch, sa, sb, bshape = _batch_layout(a_shape, b_shape, M * K, N * K, 'dev_batched_matmul_nt')
    return _gemm(1, M, N, K, batch, gt_a, sa, gt_b, K, sb, bshape + (M, N), alpha, None, SF_EPI_NONE)


def dev_matmul_tn(gt_a, gt_b, float alpha=1.0):
    """C = alpha * A^T @ B, A (K,M), B (K,N) -> (M,N): the product of
    blas_sgemm_tn (reference _mps_ops.pyx:279-298), one launch, no
    transposed copy of A."""
    _same_dtype(gt_a, gt_b, 'dev_matmul_tn')
    if len(gt_a.shape) != 2 or len(gt_b.shape) != 2:
        raise ValueError("dev_matmul_tn expects 2-D operands")
    cdef int64_t K = gt_a.shape[0], M = gt_a.shape[1], N = gt_b.shape[1]
    if gt_b.shape[0] != K:
        raise ValueError("dev_matmul_tn: shapes %s and %s not aligned" % (gt_a.shape, gt_b.shape))
    return _gemm_tn(M, N, K, 1, gt_a, 0, gt_b, 0, (M, N), alpha)


def dev_batched_matmul_tn(gt_a, gt_b, float alpha=1.0):
    """C[...] = alpha * A[...]^T @ B[...], A (...,K,M), B (...,K,N): the
    second-operand gradient of a batched matmul (reference autograd.py:296,
    np.matmul(a_T, g)), one strided-batched launch."""
    _same_dtype(gt_a, gt_b, 'dev_batched_matmul_tn')
    a_shape, b_shape = gt_a.shape, gt_b.shape
    if len(a_shape) < 2 or len(b_shape) < 2:
        raise ValueError("dev_batched_matmul_tn expects operands of rank >= 2")
    cdef int64_t K = a_shape[-2], M = a_shape[-1], N = b_shape[-1]
    if b_shape[-2] != K:
        raise ValueError("dev_batched_matmul_tn: shapes %s and %s not aligned" % (a_shape, b_shape))
    batch, sa, sb, bshape = _batch_layout(a_shape, b_shape, K * M, K * N, 'dev_batched_matmul_tn')
    return _gemm_tn(M, N, K, batch, gt_a, sa, gt_b, sb, bshape + (M, N), alpha)


def dev_sum_dim(gt, int dim=-1, bint keepdim=False):
    """Sum along dim on the device (reference :1710-1741), fp32
    accumulation, result in the input dtype."""
    shape = gt.shape
    cdef int ndim = len(shape)
    if ndim == 0:
        raise ValueError("dev_sum_dim: 0-d tensor")
    if dim < 0:
        dim += ndim
    if dim < 0 or dim >= ndim:
        raise ValueError("dev_sum_dim: dim out of range for shape %s" % (shape,))
    cdef int64_t outer = 1, inner = 1
    for i in range(dim):
        outer *= shape[i]
    cdef int64_t dim_size = shape[dim]
    for i in range(dim + 1, ndim):
        inner *= shape[i]
    out_shape = list(shape)
    if keepdim:
        out_shape[dim] = 1
    else:
        out_shape.pop(dim)
    if len(out_shape) == 0:
        out_shape = [1]
    out = _alloc_like(tuple(out_shape), gt.dtype, gt.device_id)
    cdef sf_dtype sdt = _sf_dtype(gt.dtype)
    cdef void* px = _ptr(gt)
    cdef void* po = _ptr(out)
    cdef int ret
    with nogil:
        ret = sf_sum_dim(px, po, outer, dim_size, inner, sdt, sdt, NULL)
    _check_kernel(ret)
    return out


def dev_linear_backward(gt_grad, gt_x, gt_weight, bint has_bias=True):
    """Gradients of y = x @ W^T (+ b) (reference autograd.py:793-822,
    LinearBackward.backward): grad_input = g @ W (one NN GEMM),
    grad_weight = g_2d^T @ x_2d (one TN GEMM, no transposed copy),
    grad_bias = g_2d summed over rows (None without a bias).
    g (..., N), x (..., K), W (N, K)."""
    _same_dtype(gt_grad, gt_x, 'dev_linear_backward')
    _same_dtype(gt_grad, gt_weight, 'dev_linear_backward')
    if len(gt_weight.shape) != 2 or len(gt_grad.shape) < 1 or len(gt_x.shape) < 1:
        raise ValueError("dev_linear_backward: g must be (..., N), x (..., K) and W (N, K)")
    cdef int64_t N = gt_weight.shape[0], K = gt_weight.shape[1]
    if gt_grad.shape[-1] != N or gt_x.shape[-1] != K or tuple(gt_grad.shape[:-1]) != tuple(gt_x.shape[:-1]):
        raise ValueError("dev_linear_backward: g %s, x %s and W %s not aligned"
                         % (gt_grad.shape, gt_x.shape, gt_weight.shape))
    cdef int64_t M = 1
    for s in gt_grad.shape[:-1]:
        M *= s
    grad_input = _gemm(0, M, K, N, 1, gt_grad, 0, gt_weight, K, 0, tuple(gt_x.shape), 1.0, None, SF_EPI_NONE)
    grad_weight = _gemm_tn(N, K, M, 1, gt_grad, 0, gt_x, 0, (N, K), 1.0)
    grad_bias = None
    cdef sf_dtype sdt = _sf_dtype(gt_grad.dtype)
    cdef void* pg
    cdef void* pb
    cdef int ret
    if has_bias:
        grad_bias = _alloc_like((N,), gt_grad.dtype, gt_grad.device_id)
        pg = _ptr(gt_grad)
        pb = _ptr(grad_bias)
        with nogil:
            ret = sf_sum_dim(pg, pb, 1, M, N, sdt, sdt, NULL)
        _check_kernel(ret)
    return grad_input, grad_weight, grad_bias


_ACTS = {None: 0, 'none': 0, 'silu': 1, 'gelu': 2, 'gelu_tanh': 2}


def dev_linear_forward(gt_x, gt_weight, gt_bias=None, activation=None, residual=None):
    """y = act(x @ W^T + b) (+ residual), one fused launch  (reference
    :1278-1302, which runs SGEMM then a bias pass; SiLU/GELU and the DiT
    block's residual adds, diffusion/models.py:563,588, were further passes).
    x (..., K), W (N, K), b (N,), residual (..., N) -> y (..., N)."""
    _same_dtype(gt_x, gt_weight, 'dev_linear_forward')
    if len(gt_x.shape) < 1 or len(gt_weight.shape) != 2:
        raise ValueError("dev_linear_forward: x must be (..., K) and W (N, K)")
    cdef int64_t K = gt_x.shape[-1]
    cdef int64_t N = gt_weight.shape[0]
    if gt_weight.shape[1] != K:
        raise ValueError("dev_linear_forward: x %s and W %s not aligned" % (gt_x.shape, gt_weight.shape))
    cdef int64_t M = gt_x.numel // K if K > 0 else 0
    if K == 0:
        M = 1
        for s in gt_x.shape[:-1]:
            M *= s
    if activation not in _ACTS:
        raise ValueError("dev_linear_forward: unknown activation %r" % (activation,))
    cdef int act = _ACTS[activation]
    cdef int epi
    if gt_bias is not None:
        if gt_bias.dtype != gt_x.dtype or gt_bias.numel != N:
            raise ValueError("dev_linear_forward: bias must be (%d,) of the input dtype" % N)
        epi = (SF_EPI_BIAS, SF_EPI_BIAS_SILU, SF_EPI_BIAS_GELU_TANH)[act]
    else:
        epi = (SF_EPI_NONE, SF_EPI_SILU, SF_EPI_GELU_TANH)[act]
    out_shape = tuple(gt_x.shape[:-1]) + (N,)
    if residual is not None:
        if residual.dtype != gt_x.dtype or tuple(residual.shape) != out_shape:
            raise ValueError("dev_linear_forward: residual must be %s of the input dtype, got %s"
                             % (out_shape, tuple(residual.shape)))
        if residual.device_id != gt_x.device_id:
            raise ValueError("dev_linear_forward: residual on device %d, x on %d"
                             % (residual.device_id, gt_x.device_id))
    return _gemm(1, M, N, K, 1, gt_x, 0, gt_weight, K, 0, out_shape, 1.0, gt_bias, epi, residual)


def dev_bias_add(gt_c, gt_bias):
    """In-place C[i, j] += b[j] (reference cuda_bias_add_row_f32)."""
    cdef int64_t N = gt_c.shape[-1]
    cdef int64_t M = gt_c.numel // N
    _check_kernel(sf_bias_add_rows(_ptr(gt_c), _ptr(gt_bias), M, N, _sf_dtype(gt_c.dtype), NULL))
    return gt_c


# ================================================================
#  Normalisation and residual glue (reference :965-966, :1195-1241;
#  diffusion/models.py:470-590)
# ================================================================

cdef object _need_vector(gt, int64_t n, str name):
    if gt is None:
        return None
    if gt.numel != n:
        raise ValueError("%s: expected %d elements, got shape %s" % (name, n, gt.shape))
    return gt


def dev_layer_norm(gt_x, gt_gamma=None, gt_beta=None, float eps=1e-5):
    """Layer norm over the last dim (reference :1195-1216, which takes
    (N, D) fp32; any rank and the 16-bit dtypes here, result in the input
    dtype).  gamma / beta: (D,) of the input dtype or None."""
    if len(gt_x.shape) < 1:
        raise ValueError("dev_layer_norm: scalar input")
    cdef int64_t D = gt_x.shape[-1]
    cdef int64_t rows = gt_x.numel // D if D > 0 else 0
    for g in (gt_gamma, gt_beta):
        if g is not None:
            _same_dtype(gt_x, g, 'dev_layer_norm')
    _need_vector(gt_gamma, D, 'dev_layer_norm gamma')
    _need_vector(gt_beta, D, 'dev_layer_norm beta')
    out = _alloc_like(tuple(gt_x.shape), gt_x.dtype, gt_x.device_id)
    cdef void* pg = _ptr(gt_gamma) if gt_gamma is not None else NULL
    cdef void* pb = _ptr(gt_beta) if gt_beta is not None else NULL
    cdef void* px = _ptr(gt_x)
    cdef void* py = _ptr(out)
    cdef sf_dtype dt = _sf_dtype(gt_x.dtype)
    cdef int ret
    with nogil:
        ret = sf_layer_norm(px, py, rows, D, pg, pb, eps, NULL, NULL, 0, 1, NULL, NULL, dt, NULL)
    _check_kernel(ret)
    return out


def dev_ada_layer_norm(gt_x, gt_params, float eps=1e-5, gt_gamma=None, gt_beta=None):
    """Adaptive layer norm in one launch (reference AdaLayerNorm.forward,
    diffusion/models.py:478-486): h = LayerNorm(x) (gamma, beta), then
    h * (1 + scale) + shift with scale = params[..., :C], shift =
    params[..., C:].  x (B, N, C) or (N, C); params (B, 2C), (B, 1, 2C) or
    (2C,): one row of modulation per batch entry, broadcast over its N
    tokens (the reference's NumPy broadcast does this for B == 1 and for
    params of shape (B, 1, 2C))."""
    shape = tuple(gt_x.shape)
    if len(shape) < 2:
        raise ValueError("dev_ada_layer_norm: x must be (N, C) or (B, N, C)")
    cdef int64_t C = shape[-1]
    cdef int64_t Nt = shape[-2]
    cdef int64_t B = gt_x.numel // (Nt * C) if Nt * C > 0 else 0
    _same_dtype(gt_x, gt_params, 'dev_ada_layer_norm')
    if gt_params.numel != B * 2 * C or gt_params.shape[-1] != 2 * C:
        raise ValueError("dev_ada_layer_norm: params %s do not hold one (2C,) row per batch entry of x %s"
                         % (gt_params.shape, shape))
    for g in (gt_gamma, gt_beta):
        if g is not None:
            _same_dtype(gt_x, g, 'dev_ada_layer_norm')
    _need_vector(gt_gamma, C, 'dev_ada_layer_norm gamma')
    _need_vector(gt_beta, C, 'dev_ada_layer_norm beta')
    out = _alloc_like(shape, gt_x.dtype, gt_x.device_id)
    cdef int64_t rows = B * Nt
    cdef void* pg = _ptr(gt_gamma) if gt_gamma is not None else NULL
    cdef void* pb = _ptr(gt_beta) if gt_beta is not None else NULL
    cdef void* px = _ptr(gt_x)
    cdef void* py = _ptr(out)
    cdef char* pm = <char*>_ptr(gt_params)
    cdef sf_dtype dt = _sf_dtype(gt_x.dtype)
    cdef void* pshift = pm + C * _itemsize(gt_x.dtype)
    cdef int ret
    with nogil:
        ret = sf_layer_norm(px, py, rows, C, pg, pb, eps, pm, pshift, 2 * C, Nt, NULL, NULL, dt, NULL)
    _check_kernel(ret)
    return out


def dev_rms_norm(gt_x, gt_gamma=None, float eps=1e-5):
    """RMS norm over the last dim (reference :1221-1241)."""
    if len(gt_x.shape) < 1:
        raise ValueError("dev_rms_norm: scalar input")
    cdef int64_t D = gt_x.shape[-1]
    cdef int64_t rows = gt_x.numel // D if D > 0 else 0
    if gt_gamma is not None:
        _same_dtype(gt_x, gt_gamma, 'dev_rms_norm')
    _need_vector(gt_gamma, D, 'dev_rms_norm gamma')
    out = _alloc_like(tuple(gt_x.shape), gt_x.dtype, gt_x.device_id)
    cdef void* pg = _ptr(gt_gamma) if gt_gamma is not None else NULL
    cdef void* px = _ptr(gt_x)
    cdef void* py = _ptr(out)
    cdef sf_dtype dt = _sf_dtype(gt_x.dtype)
    cdef int ret
    with nogil:
        ret = sf_rms_norm(px, py, rows, D, pg, eps, dt, NULL)
    _check_kernel(ret)
    return out


def dev_add(gt_a, gt_b):
    """a + b elementwise, equal shapes (reference :965-966)."""
    _same_dtype(gt_a, gt_b, 'dev_add')
    if tuple(gt_a.shape) != tuple(gt_b.shape):
        raise ValueError("dev_add: shapes %s and %s differ" % (gt_a.shape, gt_b.shape))
    out = _alloc_like(tuple(gt_a.shape), gt_a.dtype, gt_a.device_id)
    cdef void* pa = _ptr(gt_a)
    cdef void* pb = _ptr(gt_b)
    cdef void* py = _ptr(out)
    cdef int64_t n = gt_a.numel
    cdef sf_dtype dt = _sf_dtype(gt_a.dtype)
    cdef int ret
    with nogil:
        ret = sf_add(pa, pb, py, n, dt, NULL)
    _check_kernel(ret)
    return out


# Score memory of the unfused multi-head fallback per launch group.
_MHA_SCORES_BYTES = 1 << 30


cdef object _mha_strided(q, int64_t q_off, int64_t ldq, k, int64_t k_off, int64_t ldk,
                         v, int64_t v_off, int64_t ldv, int64_t B, int64_t Nq, int64_t Sk,
                         int64_t H, int64_t D, float scale):
    """Attention of H heads read in place from row-major [B, S, ld] operands
    (head h at column offset off + h * D), output [B, Nq, H * D]."""
    dt = q.dtype
    cdef sf_dtype sdt = _sf_dtype(dt)
    cdef int64_t C = H * D
    out = _alloc_like((B, Nq, C), dt, q.device_id)
    cdef int64_t es = _itemsize(dt)
    cdef char* pq = <char*>_ptr(q) + q_off * es
    cdef char* pk = <char*>_ptr(k) + k_off * es
    cdef char* pv = <char*>_ptr(v) + v_off * es
    cdef char* po = <char*>_ptr(out)
    cdef int ret = SF_ERR_UNSUPPORTED
    if sdt != SF_F32 and 8 <= D <= 64 and D % 8 == 0 and scale > 0:
        with nogil:
            ret = sf_attention_heads(pq, ldq, Nq * ldq, D, pk, ldk, Sk * ldk, D, pv, ldv, Sk * ldv, D,
                                     po, C, Nq * C, D, B, H, Nq, Sk, D, scale, sdt, NULL)
        if ret != SF_ERR_UNSUPPORTED:
            _check_kernel(ret)
            return out
    # Any head size, dtype or scale: per batch entry and group of heads,
    # the scores of those heads by one strided-batched NT GEMM (the scale in
    # its epilogue), the row softmax, then one strided-batched NN GEMM
    # writing the heads side by side into the output rows.  A head group's
    # scores stay within _MHA_SCORES_BYTES (at least one head).
    cdef int64_t per_head = Nq * Sk * es
    cdef int64_t hg = _MHA_SCORES_BYTES // per_head if per_head > 0 else H
    if hg < 1:
        hg = 1
    if hg > H:
        hg = H
    scores = _alloc_like((hg, Nq, Sk), dt, q.device_id)
    cdef char* ps = <char*>_ptr(scores)
    cdef int64_t b, h0, nh
    for b in range(B):
        for h0 in range(0, H, hg):
            nh = H - h0 if H - h0 < hg else hg
            with nogil:
                ret = sf_gemm(0, 1, Nq, Sk, D, nh, pq + (b * Nq * ldq + h0 * D) * es, ldq, D,
                              pk + (b * Sk * ldk + h0 * D) * es, ldk, D,
                              ps, Sk, Nq * Sk, sdt, sdt, scale, NULL, SF_EPI_NONE, NULL)
            _check_kernel(ret)
            with nogil:
                ret = sf_softmax_rows(ps, ps, nh * Nq, Sk, sdt, sdt, 1.0, NULL)
            _check_kernel(ret)
            with nogil:
                ret = sf_gemm(0, 0, Nq, D, Sk, nh, ps, Sk, Nq * Sk, pv + (b * Sk * ldv + h0 * D) * es, ldv, D,
                              po + (b * Nq * C + h0 * D) * es, C, D, sdt, sdt, 1.0, NULL, SF_EPI_NONE, NULL)
            _check_kernel(ret)
    return out


def dev_attention_packed(gt_qkv, int heads, scale=None):
    """Self-attention straight from a packed projection: qkv (B, N, 3C) ->
    (B, N, C), C = heads * D, q / k / v = qkv[..., 0:C], [C:2C], [2C:3C],
    head h at columns h*D..h*D+D-1 of each (reference DiTBlock,
    diffusion/models.py:550-559: head split, _attn, merge).  No split or
    merge copies: the fused kernel reads the heads in place and writes the
    merged rows."""
    shape = tuple(gt_qkv.shape)
    if len(shape) not in (2, 3) or shape[-1] % (3 * heads) != 0 or heads < 1:
        raise ValueError("dev_attention_packed: qkv must be (B, N, 3 * heads * D), got %s for %d heads"
                         % (shape, heads))
    cdef int64_t B = shape[0] if len(shape) == 3 else 1
    cdef int64_t N = shape[-2]
    cdef int64_t C = shape[-1] // 3
    cdef int64_t D = C // heads
    s = (1.0 / sqrt(<double>D)) if scale is None else float(scale)
    out = _mha_strided(gt_qkv, 0, 3 * C, gt_qkv, C, 3 * C, gt_qkv, 2 * C, 3 * C, B, N, N, heads, D, s)
    return out if len(shape) == 3 else dev_reshape(out, (N, C))


def dev_multihead_attention(gt_q, gt_k, gt_v, int heads, scale=None):
    """Attention over heads packed in the last dim: q (B, N, C), k and v
    (B, S, C) -> (B, N, C), C = heads * D (the reference's cross-attention,
    diffusion/models.py:566-577, without its split / merge copies)."""
    _same_dtype(gt_q, gt_k, 'dev_multihead_attention')
    _same_dtype(gt_q, gt_v, 'dev_multihead_attention')
    qs, ks, vs = tuple(gt_q.shape), tuple(gt_k.shape), tuple(gt_v.shape)
    if len(qs) != 3 or ks != vs or len(ks) != 3 or ks[0] != qs[0] or ks[2] != qs[2] or heads < 1 \
            or qs[2] % heads != 0:
        raise ValueError("dev_multihead_attention: q (B, N, C), k and v (B, S, C), C divisible by heads; "
                         "got %s %s %s" % (qs, ks, vs))
    cdef int64_t C = qs[2]
    cdef int64_t D = C // heads
    s = (1.0 / sqrt(<double>D)) if scale is None else float(scale)
    return _mha_strided(gt_q, 0, C, gt_k, 0, C, gt_v, 0, C, qs[0], qs[1], ks[1], heads, D, s)


# ================================================================
#  Elementwise / softmax (reference :944-948, :990-998, :1016-1034)
# ================================================================

def dev_silu(gt):
    out = _alloc_like(gt.shape, gt.dtype, gt.device_id)
    _check_kernel(sf_silu(_ptr(gt), _ptr(out), gt.numel, _sf_dtype(gt.dtype), NULL))
    return out


def dev_gelu(gt):
    out = _alloc_like(gt.shape, gt.dtype, gt.device_id)
    _check_kernel(sf_gelu(_ptr(gt), _ptr(out), gt.numel, _sf_dtype(gt.dtype), NULL))
    return out


def dev_muls(gt, float scalar):
    out = _alloc_like(gt.shape, gt.dtype, gt.device_id)
    _check_kernel(sf_muls(_ptr(gt), scalar, _ptr(out), gt.numel, _sf_dtype(gt.dtype), NULL))
    return out


# The random stream that dropout without an explicit seed draws from: a
# seed (manual_seed) and an offset that every draw advances, so successive
# calls get independent masks and a run is reproducible from its seed.
cdef unsigned long long _rng_seed = 0
cdef unsigned long long _rng_offset = 0


def manual_seed(unsigned long long seed):
    """Seeds the device random stream (dropout) and restarts its offsets.
    The reference's cuda.manual_seed is a no-op (cuda/__init__.py:366-368)
    and its dropout always passes seed 0 (_cuda_ops.pyx:1243)."""
    global _rng_seed, _rng_offset
    _rng_seed = seed
    _rng_offset = 0


def next_random_stream():
    """(seed, offset) for the next draw; advances the offset."""
    global _rng_offset
    cdef unsigned long long o = _rng_offset
    _rng_offset += 1
    return _rng_seed, o


def dev_dropout(gt, float p, unsigned long long seed=0, unsigned long long offset=0, bint with_mask=True):
    """Dropout on device (reference :1243-1255).  Returns (output, mask),
    both in gt's dtype: mask = 1 / (1 - p) where an element is kept (with
    probability 1 - p), else 0; output = gt * mask.  The keep decisions come
    from the Philox4x32-10 stream (seed, offset), so equal arguments give
    equal masks; the reference's stream is cuRAND's, so masks agree with it
    in law, not element for element.  with_mask=False neither allocates nor
    writes the mask and returns (output, None)."""
    if not (0.0 <= p < 1.0):
        raise ValueError("dev_dropout: p must be in [0, 1), got %r" % p)
    out = _alloc_like(gt.shape, gt.dtype, gt.device_id)
    mask = _alloc_like(gt.shape, gt.dtype, gt.device_id) if with_mask else None
    cdef void* pm = _ptr(mask) if with_mask else NULL
    _check_kernel(sf_dropout(_ptr(gt), _ptr(out), pm, gt.numel, _sf_dtype(gt.dtype), p, seed, offset, NULL))
    return out, mask


def dev_softmax(gt, int dim=-1, float scale=1.0):
    """softmax(scale * x) along the last dim."""
    cdef int ndim = len(gt.shape)
    if ndim == 0:
        raise ValueError("dev_softmax: scalar input")
    if dim != -1 and dim != ndim - 1:
        raise NotImplementedError("dev_softmax: only the last dim is supported on the device")
    cdef int64_t cols = gt.shape[ndim - 1]
    cdef int64_t rows = gt.numel // cols if cols > 0 else 0
    out = _alloc_like(gt.shape, gt.dtype, gt.device_id)
    cdef sf_dtype dt = _sf_dtype(gt.dtype)
    cdef void* px = _ptr(gt)
    cdef void* py = _ptr(out)
    cdef int ret
    with nogil:
        ret = sf_softmax_rows(px, py, rows, cols, dt, dt, scale, NULL)
    _check_kernel(ret)
    return out


def _mask_layout(tuple mshape, tuple sshape):
    """How a C-contiguous mask of shape `mshape` broadcasts (NumPy rules)
    onto scores of shape `sshape` = (..., Sq, Sk): (rows_per_batch,
    inner_batches, stride_outer, stride_inner, stride_row, stride_col) of
    sf_softmax_rows_masked.  The scores' leading dims are merged into at
    most two groups (outer, inner) of uniform mask stride; a mask that needs
    more groups raises NotImplementedError."""
    cdef int nd = len(sshape)
    if nd < 1 or len(mshape) > nd:
        raise ValueError("attn_mask of shape %s does not broadcast to scores %s" % (mshape, sshape))
    ms = (1,) * (nd - len(mshape)) + tuple(mshape)
    st = [0] * nd
    acc = 1
    for i in range(nd - 1, -1, -1):
        st[i] = acc
        acc *= ms[i]
    eff = []
    for i in range(nd):
        if ms[i] == sshape[i]:
            eff.append(st[i] if sshape[i] != 1 else 0)
        elif ms[i] == 1:
            eff.append(0)
        else:
            raise ValueError("attn_mask of shape %s does not broadcast to scores %s" % (mshape, sshape))
    s_col = eff[nd - 1]
    s_row = eff[nd - 2] if nd >= 2 else 0
    per = sshape[nd - 2] if nd >= 2 else 1
    merged = []
    for i in range(nd - 2):
        n, stv = sshape[i], eff[i]
        if n == 1:
            continue
        if merged and merged[-1][1] == n * stv:
            merged[-1] = (merged[-1][0] * n, stv)
        else:
            merged.append((n, stv))
    if len(merged) > 2:
        raise NotImplementedError("attn_mask of shape %s broadcasts over scores %s in more than two groups of "
                                  "leading dims" % (mshape, sshape))
    if not merged:
        return per, 1, 0, 0, s_row, s_col
    if len(merged) == 1:
        return per, merged[0][0], 0, merged[0][1], s_row, s_col
    return per, merged[1][0], merged[0][1], merged[1][1], s_row, s_col


def dev_softmax_masked(scores, mask, float scale=1.0):
    """softmax(scale * scores + mask) along the last dim, in place of the
    reference's host branch scores *= scale; scores += mask; softmax
    (nn/functional.py:337-347).  `mask` (a GpuTensor, or a host array that
    is uploaded as fp32) broadcasts to the scores' shape with NumPy's rules;
    additive, -inf entries allowed."""
    if not isinstance(mask, GpuTensor):
        mask = gputensor_from_numpy(np.ascontiguousarray(mask, dtype=np.float32), scores.device_id)
    if mask.device_id != scores.device_id:
        raise ValueError("dev_softmax_masked: the mask is on device %d, the scores on %d"
                         % (mask.device_id, scores.device_id))
    if mask.dtype != np.float32 and mask.dtype != scores.dtype:
        mask = dev_cast(mask, np.float32)
    sshape = tuple(scores.shape)
    if len(sshape) == 0:
        raise ValueError("dev_softmax_masked: scalar input")
    per, inner, so, si, sr, sc = _mask_layout(tuple(mask.shape), sshape)
    cdef int64_t cols = sshape[len(sshape) - 1]
    cdef int64_t rows = scores.numel // cols if cols > 0 else 0
    out = _alloc_like(sshape, scores.dtype, scores.device_id)
    cdef sf_dtype dt = _sf_dtype(scores.dtype)
    cdef sf_dtype mdt = _sf_dtype(mask.dtype)
    cdef void* px = _ptr(scores)
    cdef void* py = _ptr(out)
    cdef void* pm = _ptr(mask)
    cdef int64_t c_per = per, c_inner = inner, c_so = so, c_si = si, c_sr = sr, c_sc = sc
    cdef int ret
    with nogil:
        ret = sf_softmax_rows_masked(px, py, rows, cols, dt, scale, pm, mdt, c_per, c_inner, c_so, c_si, c_sr,
                                     c_sc, NULL)
    _check_kernel(ret)
    return out


def dev_sdpa_unfused(q, k, v, scale=None, attn_mask=None, float dropout_p=0.0, unsigned long long seed=0,
                     unsigned long long offset=0):
    """softmax(scale * Q K^T (+ attn_mask)) V in three launches (QK^T with
    the scale folded into its epilogue, row softmax with the additive mask
    folded in, PV), scores kept in the input dtype: the reference GPU path's
    structure (nn/functional.py:310-321), with the mask of its host branch
    (:339-341).  dropout_p > 0: dropout on the probabilities before PV
    (:317-318), from the random stream (seed, offset) of dev_dropout."""
    d = q.shape[-1]
    s = (1.0 / sqrt(<double>d)) if scale is None else float(scale)
    scores = dev_batched_matmul_nt(q, k, s)
    if attn_mask is None:
        probs = dev_softmax(scores, -1)
    else:
        probs = dev_softmax_masked(scores, attn_mask)
    del scores
    if dropout_p > 0.0:
        probs, _ = dev_dropout(probs, dropout_p, seed, offset, False)
    return dev_batched_matmul(probs, v)


def dev_scaled_dot_product_attention(q, k, v, scale=None, attn_mask=None, float dropout_p=0.0,
                                     unsigned long long seed=0, unsigned long long offset=0):
    """softmax(scale * Q K^T (+ attn_mask)) V  (reference GPU path
    nn/functional.py:310-321; the mask as its host branch :339-341).
    q (..., Sq, D), k and v (..., Sk, D) with equal leading dims.  One fused
    launch (sf_attention: scores never reach memory) for 16-bit inputs with
    D a multiple of 8 up to 64, a positive finite scale, no mask and no
    dropout; otherwise, or when sf_attention declines the call
    (SF_ERR_UNSUPPORTED), the three-launch path (dropout_p > 0: dev_dropout
    on the probabilities with the stream (seed, offset))."""
    d = q.shape[-1]
    s = (1.0 / sqrt(<double>d)) if scale is None else float(scale)
    _same_dtype(q, k, 'dev_scaled_dot_product_attention')
    _same_dtype(q, v, 'dev_scaled_dot_product_attention')
    if len(q.shape) < 2 or len(k.shape) != len(q.shape) or len(v.shape) != len(q.shape):
        raise ValueError("dev_scaled_dot_product_attention: q, k, v must be (..., S, D) of equal rank")
    if tuple(k.shape[:-2]) != tuple(q.shape[:-2]) or tuple(v.shape[:-2]) != tuple(q.shape[:-2]) \
            or k.shape[-1] != d or v.shape[-1] != d or v.shape[-2] != k.shape[-2]:
        raise ValueError("dev_scaled_dot_product_attention: shapes %s %s %s do not match"
                         % (q.shape, k.shape, v.shape))
    cdef int64_t sq = q.shape[-2]
    cdef int64_t sk = k.shape[-2]
    cdef int64_t batch = 1
    for e in q.shape[:-2]:
        batch *= e
    if not (0.0 <= dropout_p < 1.0):
        raise ValueError("dev_scaled_dot_product_attention: dropout_p must be in [0, 1), got %r" % dropout_p)
    if attn_mask is not None or dropout_p > 0.0 or q.dtype == np.float32 or d < 8 or d > 64 or d % 8 != 0 \
            or not (0.0 < s < 3.0e38):
        return dev_sdpa_unfused(q, k, v, scale, attn_mask, dropout_p, seed, offset)
    out = _alloc_like(tuple(q.shape), q.dtype, q.device_id)
    cdef int ret
    cdef void* pq = _ptr(q)
    cdef void* pk = _ptr(k)
    cdef void* pv = _ptr(v)
    cdef void* po = _ptr(out)
    cdef sf_dtype dt = _sf_dtype(q.dtype)
    cdef float fs = s
    cdef int64_t dh = d
    with nogil:
        ret = sf_attention(pq, dh, sq * dh, pk, dh, sk * dh, pv, dh, sk * dh, po, dh, sq * dh,
                           batch, sq, sk, dh, fs, dt, NULL)
    if ret == SF_ERR_UNSUPPORTED:
        del out
        return dev_sdpa_unfused(q, k, v, scale)
    _check_kernel(ret)
    return out


# ================================================================
#  Host-array wrappers (reference :2120-2224, :2453-2467): upload, run on
#  the device, download.
# ================================================================

def cuda_matmul(cnp.ndarray a not None, cnp.ndarray b not None):
    ga = gputensor_from_numpy(np.ascontiguousarray(a, dtype=np.float32))
    gb = gputensor_from_numpy(np.ascontiguousarray(b, dtype=np.float32))
    return gputensor_to_numpy(dev_matmul(ga, gb))


def cuda_matmul_nt(cnp.ndarray a not None, cnp.ndarray b not None):
    ga = gputensor_from_numpy(np.ascontiguousarray(a, dtype=np.float32))
    gb = gputensor_from_numpy(np.ascontiguousarray(b, dtype=np.float32))
    return gputensor_to_numpy(dev_matmul_nt(ga, gb))


def cuda_batched_matmul(cnp.ndarray a not None, cnp.ndarray b not None):
    ga = gputensor_from_numpy(np.ascontiguousarray(a, dtype=np.float32))
    gb = gputensor_from_numpy(np.ascontiguousarray(b, dtype=np.float32))
    return gputensor_to_numpy(dev_batched_matmul(ga, gb))


def cuda_linear_forward(cnp.ndarray x not None, cnp.ndarray w not None, bias=None):
    gx = gputensor_from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    gw = gputensor_from_numpy(np.ascontiguousarray(w, dtype=np.float32))
    gb = None
    if bias is not None:
        gb = gputensor_from_numpy(np.ascontiguousarray(bias, dtype=np.float32))
    return gputensor_to_numpy(dev_linear_forward(gx, gw, gb))


def library_version():
    return sf_version()


def _set_test_hooks(int xcd_shift=0, int split_spins=-1, int attn_parts=0):
    """The library's test hooks (plans forced for tests; results unchanged).
    Called with no arguments it turns them all off."""
    _check_kernel(sf_set_test_hooks(xcd_shift, split_spins, attn_parts))
