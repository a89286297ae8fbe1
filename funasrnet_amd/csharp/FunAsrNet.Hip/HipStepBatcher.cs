namespace FunAsrNet.Hip;

/// <summary>Cross-context step batching (fah_batcher_*) for the worker threads of a
/// BoundedInferencePool (BoundedInferencePool.cs:22-230) over the N FunAsr
/// contexts of SpeechRuntime (SpeechRuntime.cs:16-23): each worker's decoder
/// steps through <see cref="Step"/>, and the steps the workers request at the
/// same time run as one lock-step batch over the shared device weights.</summary>
public sealed class HipStepBatcher : IDisposable
{
    private IntPtr _batcher;

    internal HipStepBatcher(IntPtr parentDecoder, int maxPositions, int windowMicroseconds = 2000)
    {
        Native.Check(Native.fah_batcher_create(parentDecoder, maxPositions, windowMicroseconds, out _batcher));
        Owner = parentDecoder;
    }

    internal IntPtr Owner { get; }

    /// <summary>Registers a decoder whose steps the collecting thread waits for.</summary>
    internal void Join(HipDecoderStep step) => Native.Check(Native.fah_batcher_join(_batcher, step.Handle));

    internal void Leave(HipDecoderStep step) => Native.fah_batcher_leave(_batcher, step.Handle);

    /// <summary>One greedy step of <paramref name="step"/>'s decoder, batched with
    /// the other workers' concurrent steps; blocks until it has run.</summary>
    internal int Step(HipDecoderStep step)
    {
        Native.Check(Native.fah_batcher_step(_batcher, step.Handle, out int token));
        return token;
    }

    public void Dispose()
    {
        if (_batcher != IntPtr.Zero)
        {
            Native.fah_batcher_destroy(_batcher);
            _batcher = IntPtr.Zero;
        }
    }
}
