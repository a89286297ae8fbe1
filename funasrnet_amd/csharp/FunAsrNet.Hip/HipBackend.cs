using System.Runtime.CompilerServices;
using System.Runtime.InteropServices;

namespace FunAsrNet.Hip;

/// <summary>FunAsrNet backend on one HIP device (include/funasr_hip.h): Q8_0 and FP32
/// projections, grouped projections, ReLU chains, attention, and the whole Qwen3
/// decoder step. Install as the reference installs VulkanFloatBackend
/// (FunAsr.cs:66-71): <c>asr.FloatBackend = new HipBackend();</c>.</summary>
public sealed unsafe class HipBackend : IFloatComputeBackend, IQuantizedComputeBackend, IGroupedComputeBackend,
    IReluProjectionBackend, IAttentionComputeBackend, IDecoderStepBackend, IDisposable
{
    private readonly object _gate = new();                          // one stream per context (VulkanQuantizedBackend.cs:54)
    private readonly ConditionalWeakTable<Array, WeightHandle> _weights = new();  // keyed by array identity
    private readonly ConditionalWeakTable<Gguf, HipDecoderStep> _decoders = new(); // first decoder of each model
    private IntPtr _context;

    /// <param name="device">HIP device index.</param>
    /// <param name="stepBatching">Batch the concurrent decode steps of all decoders
    /// created for one model (the N contexts of a server pool) through one
    /// fah_batcher; each decoder after the first is a session over the same
    /// device weights.</param>
    public HipBackend(int device = 0, bool stepBatching = false)
    {
        Native.Check(Native.fah_context_create(device, out _context));
        StepBatching = stepBatching;
    }

    public string Name => "hip / " + (Marshal.PtrToStringUTF8(Native.fah_context_name(_context)) ?? "gfx950");
    public bool StepBatching { get; }

    /// <summary>Projections below this many multiply-adds stay on the CPU (VulkanFloatBackend.cs:36).</summary>
    public long MinimumOperations
    {
        set { lock (_gate) { Native.Check(Native.fah_context_set_minimum_operations(Live, value)); } }
    }

    private IntPtr Live
    {
        get
        {
            ObjectDisposedException.ThrowIf(_context == IntPtr.Zero, this);
            return _context;
        }
    }

    public bool TryLinear(float[] input, int frames, Weight weight, Weight? bias, float[] output)
    {
        if (weight.Values is null || weight.Quantized is not null || weight.FloatInterleaved || weight.IsTransient)
        {
            return false;
        }
        if (input.Length != checked(frames * weight.Columns) || output.Length != checked(frames * weight.Rows))
        {
            throw new ArgumentException("GPU linear projection shape mismatch");
        }
        lock (_gate)
        {
            IntPtr w = Upload(weight).Handle;
            fixed (float* x = input) fixed (float* y = output) fixed (float* b = bias?.Values)
            {
                return Native.Check(Native.fah_linear(Live, x, frames, w, b, y));
            }
        }
    }

    public bool TryConvolution(Tensor input, Tensor weight, Tensor? bias, OnnxNode node, out Tensor? output)
    {
        output = null;   // the TTS/VAD convolutions stay on the CPU
        return false;
    }

    public bool TryQuantizedLinear(float[] input, int frames, Weight weight, Weight? bias, float[] output)
    {
        if (weight.Quantized is null || weight.Scales is null || weight.QuantizedInterleaved)
        {
            return false;
        }
        if (input.Length != checked(frames * weight.Columns) || output.Length != checked(frames * weight.Rows))
        {
            throw new ArgumentException("Q8 GPU projection shape mismatch");
        }
        lock (_gate)
        {
            IntPtr w = Upload(weight).Handle;
            fixed (float* x = input) fixed (float* y = output) fixed (float* b = bias?.Values)
            {
                return Native.Check(Native.fah_quantized_linear(Live, x, frames, w, b, y));
            }
        }
    }

    public bool TryLinearMany(float[] input, int frames, Weight[] weights, out float[][]? outputs)
    {
        outputs = null;
        if (weights.Length == 0 || weights.Any(w => w.FloatInterleaved || w.QuantizedInterleaved))
        {
            return false;
        }
        lock (_gate)
        {
            var handles = new IntPtr[weights.Length];
            var result = new float[weights.Length][];              // backend-allocated (VulkanGroupedBackend.cs:49-64)
            var pins = new GCHandle[weights.Length];
            try
            {
                var pointers = new IntPtr[weights.Length];
                for (int i = 0; i < weights.Length; i++)
                {
                    handles[i] = Upload(weights[i]).Handle;
                    result[i] = new float[checked(frames * weights[i].Rows)];
                    pins[i] = GCHandle.Alloc(result[i], GCHandleType.Pinned);
                    pointers[i] = pins[i].AddrOfPinnedObject();
                }
                fixed (float* x = input) fixed (IntPtr* h = handles) fixed (IntPtr* p = pointers)
                {
                    if (!Native.Check(Native.fah_linear_many(Live, x, frames, h, weights.Length, (float**)p)))
                    {
                        return false;
                    }
                }
                outputs = result;
                return true;
            }
            finally
            {
                foreach (var pin in pins)
                {
                    if (pin.IsAllocated)
                    {
                        pin.Free();
                    }
                }
            }
        }
    }

    public bool TryReluProjection(float[] input, int frames, Weight first, Weight? firstBias, Weight second, Weight? secondBias, float[] output)
    {
        if (first.Values is null || second.Values is null || first.FloatInterleaved || second.FloatInterleaved
            || first.IsTransient || second.IsTransient)
        {
            return false;
        }
        if (input.Length != checked(frames * first.Columns) || output.Length != checked(frames * second.Rows))
        {
            throw new ArgumentException("ReLU projection input, weight or output shape mismatch");
        }
        lock (_gate)
        {
            IntPtr w1 = Upload(first).Handle, w2 = Upload(second).Handle;
            fixed (float* x = input) fixed (float* y = output) fixed (float* b1 = firstBias?.Values) fixed (float* b2 = secondBias?.Values)
            {
                return Native.Check(Native.fah_relu_projection(Live, x, frames, w1, b1, w2, b2, y));
            }
        }
    }

    public bool TryAttention(float[] query, float[] key, float[] value, int frames, int width, int heads, float[] output)
    {
        if (frames < 1 || frames > 4096 || heads < 1 || width < heads || width % heads != 0 || width / heads > 256)
        {
            return false;
        }
        int count = checked(frames * width);
        if (query.Length != count || key.Length != count || value.Length != count || output.Length != count)
        {
            throw new ArgumentException("GPU attention input/output shapes differ");
        }
        lock (_gate)
        {
            fixed (float* q = query) fixed (float* k = key) fixed (float* v = value) fixed (float* y = output)
            {
                return Native.Check(Native.fah_attention(Live, q, k, v, frames, width, heads, y));
            }
        }
    }

    public bool TryCreateDecoder(Gguf model, int capacity, out IDecoderStep? step)
    {
        step = null;
        lock (_gate)
        {
            if (StepBatching && _decoders.TryGetValue(model, out var first))
            {
                if (!first.IsDisposed)
                {
                    step = first.CreateSession(capacity);   // same device weights, own K/V
                    return true;
                }
                _decoders.Remove(model);   // its sessions keep their batcher; new decoders start afresh
            }
            var created = HipDecoderStep.Create(Live, model, capacity, StepBatching);
            if (created is null)
            {
                return false;
            }
            if (StepBatching)
            {
                _decoders.Add(model, created);
            }
            step = created;
            return true;
        }
    }

    /// <summary>Counter snapshot per seam entry point, as VulkanFloatBackend.Statistics()
    /// reports its calls, transfers and end-to-end time (VulkanFloatBackend.cs:86-118),
    /// with each kind's kernel time measured on the device.</summary>
    public object Statistics()
    {
        lock (_gate)
        {
            var stats = new Native.CallStats[Native.CallKinds.Length];
            fixed (Native.CallStats* p = stats)
            {
                Native.Check(Native.fah_context_statistics(Live, p, stats.Length));
            }
            var calls = new Dictionary<string, object>();
            for (int i = 0; i < stats.Length; i++)
            {
                var s = stats[i];
                calls[Native.CallKinds[i]] = new
                {
                    calls = s.Calls,
                    declined = s.Declined,
                    operations = s.Operations,
                    uploadedBytes = s.UploadedBytes,
                    downloadedBytes = s.DownloadedBytes,
                    deviceSeconds = s.DeviceMilliseconds / 1000.0,
                    endToEndSeconds = s.TotalMilliseconds / 1000.0,
                };
            }
            return new { device = Name, precision = "FP32 + original Q8_0", calls };
        }
    }

    /// <summary>Device copy of a weight, uploaded once per managed array
    /// (VulkanFloatBackend.cs:242-283); released with the array or the context.</summary>
    private WeightHandle Upload(Weight weight)
    {
        if (weight.Quantized is not null)
        {
            return _weights.GetValue(weight.Quantized, _ =>
            {
                fixed (sbyte* q = weight.Quantized) fixed (float* s = weight.Scales)
                {
                    Native.Check(Native.fah_weight_q8_upload(Live, q, s, weight.Rows, weight.Columns, out var h));
                    return new WeightHandle(h);
                }
            });
        }
        return _weights.GetValue(weight.Values!, _ =>
        {
            fixed (float* v = weight.Values)
            {
                Native.Check(Native.fah_weight_f32_upload(Live, v, weight.Rows, weight.Columns, out var h));
                return new WeightHandle(h);
            }
        });
    }

    /// <summary>Releases the context handle. Weights and decoders made from it stay
    /// valid to release (the library keeps the context state alive for them);
    /// calls on them report ObjectDisposedException.</summary>
    public void Dispose()
    {
        lock (_gate)
        {
            if (_context != IntPtr.Zero)
            {
                Native.fah_context_destroy(_context);
                _context = IntPtr.Zero;
            }
        }
    }
}

/// <summary>A device weight; the finalizer may run after HipBackend.Dispose,
/// which the library allows (fah_weight_release after fah_context_destroy).</summary>
internal sealed class WeightHandle(IntPtr handle)
{
    public IntPtr Handle { get; } = handle;
    ~WeightHandle() => Native.fah_weight_release(Handle);
}
