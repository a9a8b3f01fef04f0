from .synthetic_seqcls import TaskBatch, task_sampler
from .token_count import label_sequences, sample_token_count_task

__all__ = ["TaskBatch", "task_sampler", "label_sequences", "sample_token_count_task"]
