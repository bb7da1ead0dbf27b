"""The synthetic containers the golden vectors are computed on (small enough
for the reference and the oracle to run in milliseconds)."""
import container as ct

SPECS = {
    # the reference's default expert format, F32 router with bias and
    # renormalisation, Q8G group-32 shared expert
    "vq3r_f32": ct.Spec(fmt="VQ3R", router="f32", bias=True, renorm=True, routed_scale=2.0,
                        shared_bits=8, shared_group=32, seed=101),
    # 2 stages, Q8G router through mvq_rows_f32, no bias, no renormalisation,
    # Q4G group-128 shared expert
    "vq2r_q8router": ct.Spec(fmt="VQ2R", router="q8", bias=False, renorm=False, routed_scale=1.0,
                             shared_bits=4, shared_group=128, seed=102),
    # the int8-LUT format
    "vq4p_f32": ct.Spec(fmt="VQ4P", router="f32", bias=True, renorm=True, routed_scale=2.0,
                        shared_bits=8, shared_group=32, seed=103),
    # SiTU activation, Q4G router, wider top-k
    "vq3r_situ": ct.Spec(fmt="VQ3R", router="q4", bias=True, renorm=True, routed_scale=1.5,
                         act="situ", top_k=3, shared_bits=8, shared_group=32, seed=104),
    # router rows 2 and 6 identical and no bias: exact ties, lowest id wins
    "vq3r_ties": ct.Spec(fmt="VQ3R", router="f32", bias=False, renorm=True, routed_scale=1.0,
                         top_k=3, shared_bits=8, shared_group=32, dup_rows=(2, 6), seed=105),
    # K3's latent MoE: experts on a 64-wide projection of the 128-wide hidden
    # state (Q8G down/up projections, RMS norm between), Q8G shared expert
    "vq3r_latent": ct.Spec(fmt="VQ3R", router="f32", bias=True, renorm=True, routed_scale=2.5,
                           latent=64, latent_norm=True, shared_bits=8, shared_group=32, seed=106),
}
