require "../tensomite"

{% unless flag?(:hip) %}
  {% raise "tensomite/hip needs -Dhip, and libtensomite_hip.so to link against" %}
{% end %}

require "./hip/lib"

# An MI355X (gfx950) device for tensomite, over libtensomite_hip.so: the
# quantised products (`Op::BlockMatMul`) and block gathers run as the
# library's hand-written HIP kernels with the host's bits; every other op runs
# its host kernel on host copies, as on the CUDA device before an op has a
# kernel (src/tensomite/cuda.cr:395-415).
#
# Drop-in place: src/tensomite/hip.cr (with hip/lib.cr beside it), built as
#
#     LIBRARY_PATH=/path/to/tensomite.cr_amd crystal build -Dhip app.cr
#
# Written against the reference's Device/HostDevice/Node/Tensor API; not
# compiled here (no Crystal toolchain in this build's image).
module Tensomite
  # Device memory on a `HIP` GPU, with a host copy made only when a host
  # kernel reads or writes it -- the protocol `CUDABuffer` keeps
  # (cuda.cr:21-71): the device memory always holds the data; the host copy is
  # valid until the device memory is written again.
  class HIPBuffer < HostBuffer
    getter pointer : LibTensomiteHIP::DevicePtr
    @host_copy : Bytes? = nil
    @host_copy_current = false
    # Set while a host kernel writes this buffer's host copy.
    property? writing = false

    def initialize(device : HIP, @pointer : LibTensomiteHIP::DevicePtr, bytesize : Int32)
      super(device, bytesize, Bytes.empty)
    end

    # The host copy, fetched from the device when the device memory has been
    # written since (not while a host kernel is writing it).
    def bytes : Bytes
      copy = @host_copy ||= gpu.host_bytes(bytesize)
      unless @host_copy_current || writing?
        gpu.fetch(pointer, copy) unless bytesize == 0
        @host_copy_current = true
      end
      copy
    end

    # The host copy when it is current, else nil.
    def current_copy : Bytes?
      @host_copy_current ? @host_copy : nil
    end

    # A kernel or an upload wrote the device memory.
    def device_written : Nil
      @host_copy_current = false
    end

    # A host kernel wrote the host copy: it goes to the device.
    def host_written : Nil
      copy = @host_copy || raise DeviceError.new("no host copy to send to the GPU")
      gpu.store(pointer, copy) unless bytesize == 0
      @host_copy_current = true
    end

    # From a finalizer on any thread, or from #release: the host copy to the
    # device's host pool, the device memory to the library's retired list
    # (tmh_retire never waits and never raises).
    protected def give_back : Nil
      @host_copy.try { |copy| gpu.recycle(copy) }
      gpu.retire(pointer, bytesize)
    end

    private def gpu : HIP
      device.as(HIP)
    end
  end

  # An MI355X through libtensomite_hip.so. Memory is the GPU's own: `#map`
  # returns nil and data moves through `#upload` (asynchronous: the bytes are
  # copied into the library's pinned staging ring before it returns) and
  # `#download`. All work runs in submission order on one stream per GPU.
  # Any thread may call: each call makes this GPU current on the calling
  # thread first (Context#bind, cuda.cr:1118-1125).
  class HIP < HostDevice
    getter index : Int32
    getter name : String
    getter arch : String
    getter memory : UInt64
    getter compute_units : Int32

    getter uploads = 0
    getter downloads = 0
    getter gpu_ops = 0
    getter host_ops = 0

    # Where a `HIP` device's time goes, collected while `HIP#profile` is set:
    # the fields of `CUDA::Profile` (cuda.cr:249-303), so `ProfileReport` and
    # the reference's profiling benches (bench/profile_decode_cuda.cr:31-49)
    # read it as they read CUDA's.
    #
    # ```
    # hip.profile = HIP::Profile.new
    # model.forward(ids, cache)
    # hip.profile.try(&.launch) # => seconds spent launching kernels
    # ```
    class Profile
      # True when every op is timed on the GPU on its own, between two events
      # on the library's stream, waiting for it to finish: GPU time per op, at
      # the price of serialising the host and the GPU.
      getter? per_kernel : Bool

      # Count and GPU seconds per op; filled only when `#per_kernel?`.
      getter kernels = Hash(String, {Int32, Float64}).new({0, 0.0})

      # Count and wall seconds per op run on the host.
      getter host_ops = Hash(String, {Int32, Float64}).new({0, 0.0})

      # Seconds spent queuing kernels, allocating buffers, copying to and from
      # the host, and waiting for the GPU at `sync`.
      property launch = 0.0
      property alloc = 0.0
      property transfer = 0.0
      property wait = 0.0

      # Kernel launches (the library's count: a quantise pass and its product
      # are two), uploads and downloads.
      property launches = 0
      property uploads = 0
      property downloads = 0

      # Buffers allocated, those the pool could not serve, and device memory
      # freed because the pool was full.
      property allocations = 0
      property pool_misses = 0
      property frees = 0

      # True when `#kernels` keys each op by its shapes as well as its name
      # (`ProfileReport.label`); takes effect only with `#per_kernel?`.
      getter? shapes : Bool

      def initialize(@per_kernel = false, @shapes = false)
      end

      protected def add_kernel(name : String, seconds : Float64) : Nil
        count, total = kernels[name]
        kernels[name] = {count + 1, total + seconds}
      end

      protected def add_host_op(name : String, seconds : Float64) : Nil
        count, total = host_ops[name]
        host_ops[name] = {count + 1, total + seconds}
      end

      # Prints, as Markdown tables, where *wall* seconds of *runs* runs went,
      # per *unit*, from *normal* (taken as the workload ran) and the GPU
      # time per op from *timed* (`per_kernel` and `shapes`), as
      # `CUDA::Profile.report` does (cuda/report.cr:3-24).
      def self.report(io : IO, device : String, unit : String, runs : Int32, wall : Float64,
                      normal : Profile, timed : Profile, top : Int32 = 20) : Nil
        parts = [
          {"launching kernels", normal.launch},
          {"allocating buffers", normal.alloc},
          {"copying to and from the host", normal.transfer},
          {"waiting for the GPU", normal.wait},
        ]
        counts = [
          "launches: #{normal.launches // runs}; uploads: #{normal.uploads // runs}; downloads: #{normal.downloads // runs}",
          "allocations: #{normal.allocations // runs}; not from the pool: #{normal.pool_misses // runs}; freed: #{normal.frees // runs}",
        ]
        io << ProfileReport.new(device, unit, runs, wall, parts, counts, normal.host_ops, timed.kernels, top)
      end
    end

    # The profile being collected, or nil (the default) for none.
    property profile : Profile? = nil

    # The two events a per-kernel profile times each op between.
    @events : {UInt64, UInt64}? = nil

    # The library's pool of freed device memory (BufferPool, buffer_pool.cr:
    # 14-35), read through its counters: the pool itself lives in the library,
    # where finalizers on any thread give memory back without waiting.
    struct Pool
      def initialize(@gpu : HIP)
      end

      # Bytes the pool may hold: max(1 GiB, a quarter of the GPU's memory).
      def limit : Int64
        @gpu.counters.pool_limit
      end

      # Bytes of freed device memory it holds now.
      def held : Int64
        @gpu.counters.pool_held
      end

      # Allocations it served, and those it could not.
      def hits : Int64
        @gpu.counters.pool_hits
      end

      def misses : Int64
        @gpu.counters.pool_misses
      end
    end

    # The pool of freed device memory (CUDA#buffer_pool, cuda.cr:208-211).
    def buffer_pool : Pool
      Pool.new(self)
    end

    # Bytes of device memory allocated from the runtime and not yet freed: in
    # live buffers and in `#buffer_pool` (CUDA#device_bytes, cuda.cr:217-222).
    def device_bytes : Int64
      counters.device_bytes
    end

    # How a quantised matmul divides its work (BlockMatMulMode, quant.cr:5-57);
    # its value is the library's TMH_MODE_* number.
    property block_mode = BlockMatMulMode.from_env

    # The first GPU's device; raises DeviceError when there is none.
    class_getter default : HIP { HIP.new(0) }

    # GPUs the library sees (tmh_init also sets every one up).
    def self.count : Int32
      check(LibTensomiteHIP.init(out count), "tmh_init")
      count
    end

    # True when the library starts and sees a GPU; never raises, as
    # CUDA.available? (cuda.cr:986-988) for the specs' device list.
    def self.available? : Bool
      LibTensomiteHIP.init(out count) == LibTensomiteHIP::SUCCESS && count > 0
    end

    # Raises the reference's error for a failed call, "call: NAME (text)"
    # (CUDA.check, cuda.cr:1070-1075): shape and dtype codes as ShapeError and
    # DTypeError, everything else as DeviceError.
    def self.check(code : Int32, call : String) : Nil
      return if code == LibTensomiteHIP::SUCCESS
      text = "#{call}: #{String.new(LibTensomiteHIP.error_name(code))} (#{String.new(LibTensomiteHIP.error_string(code))})"
      case code
      when LibTensomiteHIP::ERROR_SHAPE then raise ShapeError.new(text)
      when LibTensomiteHIP::ERROR_DTYPE then raise DTypeError.new(text)
      else                                   raise DeviceError.new(text)
      end
    end

    def initialize(@index : Int32 = 0)
      count = HIP.count
      unless @index >= 0 && @index < count
        raise DeviceError.new("no HIP GPU #{@index} (#{count} found)")
      end
      HIP.check(LibTensomiteHIP.device_info(@index, out info), "tmh_device_info_get")
      @name = String.new(info.name.to_unsafe)
      @arch = String.new(info.arch.to_unsafe)
      @memory = info.memory
      @compute_units = info.compute_units
      bind
    end

    # Device memory of exactly *bytesize* bytes, from the library's pool when
    # a buffer of that size is free (CUDA#alloc, cuda.cr:339-353).
    def alloc(bytesize : Int32) : Buffer
      bind
      profile = @profile
      misses = profile ? counters.pool_misses : 0_i64
      start = Time.instant
      HIP.check(LibTensomiteHIP.alloc(out pointer, bytesize.to_u64), "tmh_alloc")
      if profile
        profile.alloc += (Time.instant - start).total_seconds
        profile.allocations += 1
        profile.pool_misses += 1 if counters.pool_misses > misses
      end
      HIPBuffer.new(self, pointer, bytesize)
    end

    def map(buffer : Buffer) : Bytes?
      gpu_buffer(buffer)
      nil
    end

    def upload(buffer : Buffer, data : Bytes) : Nil
      target = gpu_buffer(buffer)
      @uploads += 1
      start = Time.instant
      unless data.empty?
        bind
        HIP.check(LibTensomiteHIP.upload_async(target.pointer, data.to_unsafe, data.size.to_u64), "tmh_upload_async")
      end
      target.device_written
      @profile.try do |profile|
        profile.uploads += 1
        profile.transfer += (Time.instant - start).total_seconds
      end
    end

    def download(buffer : Buffer, data : Bytes) : Nil
      source = gpu_buffer(buffer)
      @downloads += 1
      start = Time.instant
      if copy = source.current_copy
        copy[0, data.size].copy_to(data)
      elsif !data.empty?
        fetch(source.pointer, data)
      end
      @profile.try do |profile|
        profile.downloads += 1
        profile.transfer += (Time.instant - start).total_seconds
      end
    end

    # A file mapping cannot be shared with the GPU: its bytes are copied.
    def adopt(bytes : Bytes, owner : MappedFile) : Buffer
      alloc(bytes.size).tap { |buffer| upload(buffer, bytes) }
    end

    # Queues the library's kernels for a block product or block gather; any
    # other op runs its host kernel on host copies of its sources, and its
    # output is sent to the device (cuda.cr:395-415).
    def execute(node : Node, output : Buffer) : Nil
      target = gpu_buffer(output)
      if launch_profiled(node, target)
        target.device_written
        @gpu_ops += 1
        return
      end
      start = Time.instant
      # A write keeps the rest of its target: its host copy must be current.
      target.bytes if node.op.try(&.in_place?)
      target.writing = true
      begin
        super
      ensure
        target.writing = false
      end
      target.host_written
      @host_ops += 1
      @profile.try(&.add_host_op("#{node.op} #{node.dtype}", (Time.instant - start).total_seconds))
    end

    # Waits for the GPU, moves retired memory into the pool, and raises
    # ExecutionError for a gather id a kernel found out of range
    # (CUDA#sync and #check_errors, cuda.cr:419-428, 972-983).
    def sync : Nil
      bind
      profile = @profile
      frees = profile ? counters.frees : 0_i64
      start = Time.instant
      code = LibTensomiteHIP.sync
      if profile
        profile.wait += (Time.instant - start).total_seconds
        profile.frees += (counters.frees - frees).to_i32
      end
      if code == LibTensomiteHIP::ERROR_EXECUTION
        report = StaticArray(Int32, 3).new(0)
        LibTensomiteHIP.error_report(report.to_unsafe)
        raise ExecutionError.new("index #{report[1]} out of range for #{report[2]} rows")
      end
      HIP.check(code, "tmh_sync")
    end

    # The library's counters: uploads, downloads, GPU ops, device bytes and
    # the pool's hits, misses and held bytes (cuda.cr:214-230).
    def counters : LibTensomiteHIP::Counters
      bind
      HIP.check(LibTensomiteHIP.counters(out result), "tmh_counters_get")
      result
    end

    # :nodoc:
    def host_bytes(bytesize : Int32) : Bytes
      pool.take(bytesize) || Bytes.new(bytesize)
    end

    protected def fetch(pointer : LibTensomiteHIP::DevicePtr, data : Bytes) : Nil
      bind
      HIP.check(LibTensomiteHIP.download(data.to_unsafe, pointer, data.size.to_u64), "tmh_download")
    end

    protected def store(pointer : LibTensomiteHIP::DevicePtr, data : Bytes) : Nil
      bind
      HIP.check(LibTensomiteHIP.upload(pointer, data.to_unsafe, data.size.to_u64), "tmh_upload")
    end

    # Never waits and never raises: finalizers call it on any thread. (The
    # library counts memory it frees here because its retired list was busy
    # or full; a profile picks that count up at the next `sync`.)
    protected def retire(pointer : LibTensomiteHIP::DevicePtr, bytesize : Int32) : Nil
      LibTensomiteHIP.set_device(@index)
      LibTensomiteHIP.retire(pointer, bytesize.to_u64)
    end

    # Launches *node* as `#launch_blocks` does, recording the time it takes
    # and the kernels it queued with a profile, and, with a per-kernel
    # profile, its GPU time between two events (CUDA#launch_profiled,
    # cuda.cr:461-481).
    private def launch_profiled(node : Node, output : HIPBuffer) : Bool
      return launch_blocks(node, output) unless profile = @profile
      bind
      events = @events ||= {new_event, new_event}
      HIP.check(LibTensomiteHIP.event_record(events[0]), "tmh_event_record") if profile.per_kernel?
      launches = counters.launches
      start = Time.instant
      launched = launch_blocks(node, output)
      profile.launch += (Time.instant - start).total_seconds
      profile.launches += (counters.launches - launches).to_i32
      if launched && profile.per_kernel?
        HIP.check(LibTensomiteHIP.event_record(events[1]), "tmh_event_record")
        HIP.check(LibTensomiteHIP.event_elapsed_ms(events[0], events[1], out ms), "tmh_event_elapsed_ms")
        profile.add_kernel(ProfileReport.label(node, profile.shapes?), ms / 1000.0)
      end
      launched
    end

    private def new_event : UInt64
      HIP.check(LibTensomiteHIP.event_create(out event), "tmh_event_create")
      event
    end

    private def bind : Nil
      HIP.check(LibTensomiteHIP.set_device(@index), "tmh_set_device")
    end

    private def gpu_buffer(buffer : Buffer) : HIPBuffer
      own(buffer).as?(HIPBuffer) || raise DeviceError.new("buffer is not a HIP buffer")
    end

    private def pointer(tensor : Tensor) : LibTensomiteHIP::DevicePtr
      gpu_buffer(tensor.node.buffer!).pointer
    end

    private def kind(dtype : DType) : UInt32
      case dtype
      when .q8_0? then LibTensomiteHIP::Q8_0
      when .q4_0? then LibTensomiteHIP::Q4_0
      when .q4_1? then LibTensomiteHIP::Q4_1
      else             raise DTypeError.new("#{dtype} is not a block format")
      end
    end

    # The distance in floats between consecutive rows of k values of *x*, when
    # its view is rows of k contiguous values evenly spaced (dense, or a 2-D
    # view of whole rows); else nil, and the op takes the host path, which
    # reads any view (HostDevice#activations, host.cr:675-692).
    private def row_stride(x : Tensor, k : Int32) : Int32?
      view = x.view
      return k if view.dense?
      return nil unless view.ndim == 2 && view.strides[1] == 1 && view.strides[0] >= k
      view.strides[0]
    end

    # Queues BlockMatMul (quantise pass + product, tmh_block_matmul) or a
    # block-table Gather (tmh_gather_blocks) and returns true; false for any
    # other op, for an input view the library does not read, or when the
    # library's kernels are unavailable (TMH_ERROR_NO_KERNELS, as CUDA falls
    # back when its module cannot load, cuda.cr:1164-1172).
    private def launch_blocks(node : Node, output : HIPBuffer) : Bool
      return false unless node.dtype.f32? && node.reads_blocks?
      bind
      case node.op
      when Op::BlockMatMul
        x, w = node.srcs[0], node.srcs[1]
        n, k = w.shape[0], w.shape[1]
        ldx = row_stride(x, k)
        return false unless ldx
        bias = 0_u64
        if b = node.srcs[2]?
          return false unless b.view.dense?
          bias = pointer(b) + 4_u64 * b.view.offset
        end
        code = LibTensomiteHIP.block_matmul(kind(w.dtype), pointer(w), w.dtype.bytes_for(w.view.offset).to_u64,
          pointer(x) + 4_u64 * x.view.offset, ldx.to_u32, output.pointer, bias,
          (x.size // k).to_u32, n.to_u32, k.to_u32, block_mode.value.to_u32)
        return false if code == LibTensomiteHIP::ERROR_NO_KERNELS
        HIP.check(code, "tmh_block_matmul")
      when Op::Gather
        table, ids = node.srcs[0], node.srcs[1]
        return false unless ids.view.dense?
        rows, width = table.shape[0], table.shape[1]
        code = LibTensomiteHIP.gather_blocks(kind(table.dtype), pointer(table),
          table.dtype.bytes_for(table.view.offset).to_u64, rows, width.to_u32,
          pointer(ids) + 4_u64 * ids.view.offset, ids.size.to_u32, output.pointer)
        return false if code == LibTensomiteHIP::ERROR_NO_KERNELS
        HIP.check(code, "tmh_gather_blocks")
      else
        return false
      end
      true
    end
  end

  # A Llama decoded entirely on a HIP GPU (tmh_llama_*): Llama#forward /
  # #forward_last and Generative#generate with Sampler.greedy
  # (llama.cr:256-303, generative.cr:155-190) over `rows` sequences, each
  # with its own KV cache row. Loaded straight from a GGUF file: the q/k rows
  # are unpermuted and the projections merged on the host while staging
  # (Llama.load, llama.cr:184-235), so nothing is downloaded and sent again.
  class HIPDecoder
    getter config : LibTensomiteHIP::LlamaConfig
    getter rows : Int32
    @model : UInt64

    # *capacity* 0 means the model's context.
    def initialize(@gpu : HIP, path : String, @rows : Int32 = 1, capacity : Int32 = 0, max_tokens : Int32 = 128)
      LibTensomiteHIP.set_device(@gpu.index)
      HIP.check(LibTensomiteHIP.llama_load_gguf(path.to_unsafe, @rows.to_u32, capacity.to_u32, max_tokens.to_u32,
        out config, out model), "tmh_llama_load_gguf")
      @config = config
      @model = model
    end

    # Runs *ids* in row *row* after its cached positions; returns the logits
    # of every position, or of the last one with *last_only*.
    def forward(ids : Array(Int32), row : Int32 = 0, last_only : Bool = false) : Array(Float32)
      LibTensomiteHIP.set_device(@gpu.index)
      logits = Array(Float32).new((last_only ? 1 : ids.size) * @config.vocab, 0.0_f32)
      HIP.check(LibTensomiteHIP.llama_forward(@model, row.to_u32, ids.to_unsafe, ids.size.to_u32,
        last_only ? 1_u32 : 0_u32, logits.to_unsafe), "tmh_llama_forward")
      logits
    end

    # *steps* greedy tokens for every row from its last forward's logits,
    # each decode step one replay of a captured HIP graph: tokens[row] is
    # Generative#generate's output for that row alone.
    def generate(steps : Int32, graph : Bool = true) : Array(Array(Int32))
      LibTensomiteHIP.set_device(@gpu.index)
      tokens = Array(Int32).new(@rows * steps, 0)
      HIP.check(LibTensomiteHIP.llama_generate(@model, steps.to_u32, tokens.to_unsafe, graph ? 1_u32 : 0_u32),
        "tmh_llama_generate")
      Array.new(@rows) { |r| tokens[r * steps, steps] }
    end

    def reset(row : Int32) : Nil
      HIP.check(LibTensomiteHIP.llama_reset(@model, row.to_u32), "tmh_llama_reset")
    end

    def finalize
      LibTensomiteHIP.llama_destroy(@model)
    end
  end
end
