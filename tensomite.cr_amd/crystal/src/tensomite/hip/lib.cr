# The C ABI of libtensomite_hip.so (include/tensomite_hip.h), one `fun` per
# entry point: the seam `lib LibCUDA` / `lib LibNVRTC` is for the CUDA device
# (src/tensomite/cuda/lib.cr:48-110). Results are Int32 codes (0 success,
# 1..999 HIP runtime codes, 1000+ the library's own); device memory is a
# UInt64 address; sizes in bytes are UInt64. Kernels are built offline for
# gfx950, so nothing here compiles at run time (no NVRTC counterpart).
#
# Drop-in place: src/tensomite/hip/lib.cr, linked with `-Dhip` and
# LIBRARY_PATH naming the directory of libtensomite_hip.so.
module Tensomite
  @[Link("tensomite_hip")]
  lib LibTensomiteHIP
    alias DevicePtr = UInt64

    SUCCESS              =    0
    ERROR_INVALID_VALUE  = 1000
    ERROR_SHAPE          = 1001
    ERROR_DTYPE          = 1002
    ERROR_NO_KERNELS     = 1003
    ERROR_OUT_OF_MEMORY  = 1004
    ERROR_EXECUTION      = 1005
    ERROR_NO_DEVICE      = 1006
    ERROR_BUSY           = 1007
    ERROR_NOT_READY      = 1008
    ERROR_SCRATCH_LIMIT  = 1009
    FIXED_SCRATCH_BYTES  = 8_u32 << 20

    Q8_0 = 0_u32
    Q4_0 = 1_u32
    Q4_1 = 2_u32

    X_F32       = 0_u32
    X_RMSNORM   = 1_u32
    X_QUANTISED = 2_u32

    struct DeviceInfo
      name : UInt8[256]
      arch : UInt8[64]
      memory : UInt64
      compute_units : Int32
      clock_khz : Int32
      memory_clock_khz : Int32
      memory_bus_width : Int32
      l2_bytes : Int32
      lds_bytes_per_block : Int32
    end

    struct Counters
      uploads : Int64
      downloads : Int64
      gpu_ops : Int64
      device_bytes : Int64
      pool_held : Int64
      pool_limit : Int64
      pool_hits : Int64
      pool_misses : Int64
      frees : Int64
      launches : Int64
    end

    struct Product
      w : DevicePtr
      w_byte_offset : UInt64
      x : DevicePtr
      dst : DevicePtr
      bias : DevicePtr
      n : UInt32
      k : UInt32
      x_mode : UInt32
      eps : Float32
      norm : DevicePtr
      scales : DevicePtr
      sums : DevicePtr
      totals : DevicePtr
    end

    struct LlamaConfig
      layers : Int32
      width : Int32
      heads : Int32
      kv_heads : Int32
      head_width : Int32
      hidden : Int32
      vocab : Int32
      context : Int32
      eps : Float32
      theta : Float64
      kind : UInt32
    end

    struct LlamaWeights
      embed : DevicePtr
      head : DevicePtr
      norm : DevicePtr
      attn_norm : DevicePtr*
      ffn_norm : DevicePtr*
      qkv : DevicePtr*
      o : DevicePtr*
      gate_up : DevicePtr*
      down : DevicePtr*
    end

    # devices
    fun init = tmh_init(count : Int32*) : Int32
    fun device_info = tmh_device_info_get(device : Int32, info : DeviceInfo*) : Int32
    fun set_device = tmh_set_device(device : Int32) : Int32
    fun get_device = tmh_get_device(device : Int32*) : Int32

    # memory
    fun malloc = tmh_malloc(ptr : DevicePtr*, bytes : UInt64) : Int32
    fun free = tmh_free(ptr : DevicePtr) : Int32
    fun free_any_thread = tmh_free_any_thread(ptr : DevicePtr) : Int32
    fun upload = tmh_upload(dst : DevicePtr, src : Void*, bytes : UInt64) : Int32
    fun upload_async = tmh_upload_async(dst : DevicePtr, src : Void*, bytes : UInt64) : Int32
    fun download = tmh_download(dst : Void*, src : DevicePtr, bytes : UInt64) : Int32
    fun copy = tmh_copy(dst : DevicePtr, src : DevicePtr, bytes : UInt64) : Int32
    fun synchronize = tmh_synchronize : Int32

    # the buffer layer
    fun alloc = tmh_alloc(ptr : DevicePtr*, bytes : UInt64) : Int32
    fun retire = tmh_retire(ptr : DevicePtr, bytes : UInt64) : Int32
    fun sync = tmh_sync : Int32
    fun pool_set_limit = tmh_pool_set_limit(bytes : Int64) : Int32
    fun counters = tmh_counters_get(result : Counters*) : Int32

    # errors and test hooks
    fun error_name = tmh_error_name(code : Int32) : UInt8*
    fun error_string = tmh_error_string(code : Int32) : UInt8*
    fun error_report = tmh_error_report(report : Int32*) : Int32
    fun debug_fail_allocations = tmh_debug_fail_allocations(count : Int32) : Int32
    fun debug_disable_kernels = tmh_debug_disable_kernels(off : Int32) : Int32
    fun debug_f16_words = tmh_debug_f16_words(first : UInt32, count : UInt32, dst : DevicePtr) : Int32
    fun debug_read = tmh_debug_read(src : DevicePtr, bytes : UInt64, workgroups : UInt32, out : DevicePtr) : Int32

    # events
    fun event_create = tmh_event_create(event : UInt64*) : Int32
    fun event_record = tmh_event_record(event : UInt64) : Int32
    fun event_elapsed_ms = tmh_event_elapsed_ms(start : UInt64, stop : UInt64, ms : Float32*) : Int32
    fun event_destroy = tmh_event_destroy(event : UInt64) : Int32

    # kernels
    fun quantize_rows_q8 = tmh_quantize_rows_q8(x : DevicePtr, rows : UInt32, k : UInt32, ldx : UInt32,
                                                scales : DevicePtr, sums : DevicePtr, totals : DevicePtr,
                                                qs : DevicePtr) : Int32
    fun block_matmul = tmh_block_matmul(kind : UInt32, w : DevicePtr, w_byte_offset : UInt64, x : DevicePtr,
                                        ldx : UInt32, dst : DevicePtr, bias : DevicePtr, rows : UInt32, n : UInt32,
                                        k : UInt32, mode : UInt32) : Int32
    fun block_matmul_fixed = tmh_block_matmul_fixed(kind : UInt32, w : DevicePtr, w_byte_offset : UInt64,
                                                    x : DevicePtr, ldx : UInt32, dst : DevicePtr, bias : DevicePtr,
                                                    rows : UInt32, n : UInt32, k : UInt32, mode : UInt32) : Int32
    fun block_matmul_quantised = tmh_block_matmul_quantised(kind : UInt32, w : DevicePtr, w_byte_offset : UInt64,
                                                            scales : DevicePtr, sums : DevicePtr, totals : DevicePtr,
                                                            qs : DevicePtr, dst : DevicePtr, bias : DevicePtr,
                                                            rows : UInt32, n : UInt32, k : UInt32,
                                                            mode : UInt32) : Int32
    fun gather_blocks = tmh_gather_blocks(kind : UInt32, table : DevicePtr, table_byte_offset : UInt64,
                                          table_rows : Int32, width : UInt32, ids : DevicePtr, count : UInt32,
                                          dst : DevicePtr) : Int32
    fun quantize_weights = tmh_quantize_weights(kind : UInt32, values : Float32*, count : UInt64, blocks : UInt8*,
                                                threads : Int32) : Int32

    # plans: many one-row products as one launch
    fun plan_create = tmh_plan_create(kind : UInt32, products : Product*, count : UInt32, plan : UInt64*) : Int32
    fun plan_run = tmh_plan_run(plan : UInt64) : Int32
    fun plan_destroy = tmh_plan_destroy(plan : UInt64) : Int32
    fun plan_describe = tmh_plan_describe(plan : UInt64, text : UInt8*, size : UInt32) : Int32
    fun plan_set_mode = tmh_plan_set_mode(plan : UInt64, mode : UInt32) : Int32

    # the rest of the decode graph, with the host kernels' bits
    fun rmsnorm = tmh_rmsnorm(x : DevicePtr, ldx : UInt32, weight : DevicePtr, rows : UInt32, n : UInt32,
                              eps : Float32, dst : DevicePtr) : Int32
    fun rope_write = tmh_rope_write(x : DevicePtr, ldx : UInt32, tokens : UInt32, heads : UInt32,
                                    kv_heads : UInt32, width : UInt32, cos : DevicePtr, sin : DevicePtr,
                                    table_rows : UInt32, slots : DevicePtr, cache_rows : UInt32,
                                    capacity : UInt32, q_dst : DevicePtr, keys : DevicePtr,
                                    values : DevicePtr) : Int32
    fun attention = tmh_attention(q : DevicePtr, ldq : UInt32, tokens : UInt32, heads : UInt32, keys : DevicePtr,
                                  values : DevicePtr, cache_rows : UInt32, kv_heads : UInt32, capacity : UInt32,
                                  width : UInt32, table : DevicePtr, scale : Float32, dst : DevicePtr,
                                  ld_dst : UInt32) : Int32
    fun swiglu = tmh_swiglu(gate : DevicePtr, value : DevicePtr, ld : UInt32, rows : UInt32, n : UInt32,
                            dst : DevicePtr) : Int32
    fun add = tmh_add(a : DevicePtr, b : DevicePtr, dst : DevicePtr, count : UInt64) : Int32
    fun argmax = tmh_argmax(x : DevicePtr, ldx : UInt32, rows : UInt32, n : UInt32, ids : DevicePtr) : Int32

    # the device-resident Llama decoder
    fun llama_create = tmh_llama_create(config : LlamaConfig*, weights : LlamaWeights*, rows : UInt32,
                                        capacity : UInt32, max_tokens : UInt32, model : UInt64*) : Int32
    fun llama_forward = tmh_llama_forward(model : UInt64, row : UInt32, ids : Int32*, count : UInt32,
                                          last_only : UInt32, logits : Float32*) : Int32
    fun llama_generate = tmh_llama_generate(model : UInt64, steps : UInt32, tokens : Int32*, graph : UInt32) : Int32
    fun llama_length = tmh_llama_length(model : UInt64, row : UInt32, length : Int32*) : Int32
    fun llama_reset = tmh_llama_reset(model : UInt64, row : UInt32) : Int32
    fun llama_step = tmh_llama_step(model : UInt64, graph : UInt32) : Int32
    fun llama_set_mode = tmh_llama_set_mode(model : UInt64, mode : UInt32) : Int32
    fun llama_destroy = tmh_llama_destroy(model : UInt64) : Int32

    # GGUF files
    fun gguf_open = tmh_gguf_open(path : UInt8*, file : UInt64*) : Int32
    fun gguf_close = tmh_gguf_close(file : UInt64) : Int32
    fun gguf_tensor = tmh_gguf_tensor(file : UInt64, name : UInt8*, kind : UInt32*, shape : Int64*, dims : UInt32*,
                                      bytes : UInt64*) : Int32
    fun gguf_upload = tmh_gguf_upload(file : UInt64, name : UInt8*, rows : Int32*, count : UInt32,
                                      dst : DevicePtr) : Int32
    fun llama_load_gguf = tmh_llama_load_gguf(path : UInt8*, rows : UInt32, capacity : UInt32,
                                              max_tokens : UInt32, config : LlamaConfig*, model : UInt64*) : Int32
  end
end
