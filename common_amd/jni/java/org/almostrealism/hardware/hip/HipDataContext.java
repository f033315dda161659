/*
 * DataContext for one MI355X GPU (base/code/src/main/java/io/almostrealism/code/DataContext.java:
 * 39-130, through HardwareDataContext), created by Hardware when AR_HARDWARE_DRIVER names "hip"
 * (ComputeRequirement.HIP; see the DriverSelection / Hardware changes documented with this binding).
 *
 * What it provides: device memory (HipMemoryProvider, fp32 elements), a compute context that
 * orders copies on the GPU's stream, and the native context handle that the HIP Qwen3 fast path
 * (HipQwen3) runs on.  It does not compile generated scopes: HipComputeContext.deliver refuses
 * them, and every operation other than the Qwen3 decode / prefill step stays on the CPU contexts
 * that Hardware creates beside this one.
 *
 * Not compiled in this repository (no JDK in the build image).
 */
package org.almostrealism.hardware.hip;

import io.almostrealism.code.ComputeContext;
import io.almostrealism.code.Memory;
import io.almostrealism.code.MemoryProvider;
import io.almostrealism.code.Precision;
import io.almostrealism.compute.ComputeRequirement;
import org.almostrealism.hardware.HardwareException;
import org.almostrealism.hardware.MemoryData;
import org.almostrealism.hardware.ctx.HardwareDataContext;

import java.util.List;
import java.util.concurrent.Callable;
import java.util.function.IntFunction;

public class HipDataContext extends HardwareDataContext {
	private final int device;
	private long handle;
	private HipMemoryProvider ram;
	private HipComputeContext compute;

	/**
	 * @param name            context name ("HIP")
	 * @param maxReservation  most elements the provider may hold at once (Hardware's reservation)
	 * @param device          GPU ordinal, or -1 for the one AR_HIP_DEVICE names (default 0)
	 */
	public HipDataContext(String name, long maxReservation, int device) {
		super(name, maxReservation);
		this.device = device;
	}

	/** The device arithmetic is fp32 (bf16 is a weight storage format only). */
	@Override
	public Precision getPrecision() { return Precision.FP32; }

	@Override
	public synchronized void init() {
		if (handle != 0) return;
		if (HIP.deviceCount() <= 0) {
			throw new HardwareException("HIP: no device (AR_HIP_ERR_NO_DEVICE)");
		}
		handle = HIP.init(device);
		long hbm = HIP.hbmBytes(handle);
		long max = Math.min(hbm, getMaxReservation() * (long) getPrecision().bytes());
		ram = new HipMemoryProvider(this, getPrecision().bytes(), max);
		compute = new HipComputeContext(this);
	}

	/** Native ar_hip_ctx handle (0 before init / after destroy). */
	public long getHandle() {
		if (handle == 0) throw new IllegalStateException("HIP context is not initialized");
		return handle;
	}

	public int getComputeUnits() { return HIP.computeUnits(getHandle()); }

	public String getDeviceName() { return HIP.deviceName(getHandle()); }

	@Override
	public List<MemoryProvider<? extends Memory>> getMemoryProviders() { return List.of(ram); }

	@Override
	public MemoryProvider<? extends Memory> getMemoryProvider(int size) {
		IntFunction<MemoryProvider<?>> supply = getMemoryProviderSupply();
		return supply == null ? ram : (MemoryProvider<? extends Memory>) supply.apply(size);
	}

	@Override
	public MemoryProvider<? extends Memory> getKernelMemoryProvider() { return ram; }

	@Override
	public List<ComputeContext<MemoryData>> getComputeContexts() { return List.of(compute); }

	/** Runs exec with this context's device memory as the provider for new allocations. */
	@Override
	public <T> T deviceMemory(Callable<T> exec) {
		IntFunction<MemoryProvider<?>> current = memoryProvider.get();
		try {
			memoryProvider.set(s -> ram);
			return exec.call();
		} catch (RuntimeException e) {
			throw e;
		} catch (Exception e) {
			throw new RuntimeException(e);
		} finally {
			memoryProvider.set(current);
		}
	}

	/**
	 * One stream per GPU: every expectation resolves to the same compute context (kernel work of
	 * this backend is ordered on that stream), so exec simply runs.
	 */
	@Override
	public <T> T computeContext(Callable<T> exec, ComputeRequirement... expectations) {
		for (ComputeRequirement r : expectations) {
			if (r == ComputeRequirement.CPU || r == ComputeRequirement.JNI || r == ComputeRequirement.C) {
				throw new IllegalArgumentException("HIP context cannot satisfy " + r);
			}
		}
		try {
			return exec.call();
		} catch (RuntimeException e) {
			throw e;
		} catch (Exception e) {
			throw new RuntimeException(e);
		}
	}

	@Override
	public synchronized void destroy() {
		if (handle == 0) return;
		if (compute != null) compute.destroy();
		if (ram != null) ram.destroy();
		HIP.destroy(handle);
		handle = 0;
		compute = null;
		ram = null;
	}
}
